"""PyTorch restatement of paged decode attention (the CPU baseline; the GPU
tests' full-size reference) — TEST AND BASELINE INFRASTRUCTURE ONLY.

bench.py times this as the CPU baseline of the decode path (fp32 compute on
fp16 pages, torch's intra-op threads on the host cores); tests/test_oracle.py
checks it against the numpy oracle, and the GPU tests run it on the device as
the full-size reference of the decode kernels. The product path
(kunserve_amd) never imports it.

It restates the same semantics as oracle.paged_attention_ref.decode_attention
(LlamaOp.pforward decode rows, kunserve/worker.py:298-312; pages of
kunserve/block_manager.py:786-795; heads kunserve/models.py:55-56): for each
row, gather its kv_len tokens through the page table, then
softmax(q . K^T * sm_scale) . V per query head, with query head h reading KV
head h // (Hq / Hkv).
"""
from __future__ import annotations

import numpy as np
import torch


def decode_attention(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor, layer: int,
                     indptr: np.ndarray, indices: np.ndarray, kv_len: np.ndarray,
                     sm_scale: float) -> torch.Tensor:
    """q [B, Hq, D] and pools [pages, L, Hkv, page_size, D] (any float dtype)
    on one device; returns [B, Hq, D] float32 there. A row with kv_len 0
    yields zeros. The tests also run it on the GPU, as the full-size
    reference of the decode kernels."""
    B, hq, d = q.shape
    hkv, ps = k_pool.shape[2], k_pool.shape[3]
    g = hq // hkv
    out = torch.zeros((B, hq, d), dtype=torch.float32, device=q.device)
    idx = torch.from_numpy(np.asarray(indices, dtype=np.int64)).to(k_pool.device)
    for b in range(B):
        n = int(kv_len[b])
        if n == 0:
            continue
        pages = idx[int(indptr[b]):int(indptr[b]) + (n + ps - 1) // ps]
        # [pages, Hkv, ps, D] -> [Hkv, pages * ps, D], first n tokens
        k = k_pool[pages, layer].float().transpose(0, 1).reshape(hkv, -1, d)[:, :n]
        v = v_pool[pages, layer].float().transpose(0, 1).reshape(hkv, -1, d)[:, :n]
        qb = q[b].float().reshape(hkv, g, d)
        s = torch.bmm(qb, k.transpose(1, 2).contiguous()) * sm_scale   # [Hkv, G, n]
        out[b] = torch.bmm(torch.softmax(s, dim=-1), v.contiguous()).reshape(hq, d)
    return out
