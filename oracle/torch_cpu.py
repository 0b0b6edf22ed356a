"""PyTorch restatement of paged decode and chunked-prefill attention and of
the block copy (the CPU baselines; the GPU tests' full-size reference) —
TEST AND BASELINE INFRASTRUCTURE ONLY.

bench.py times these as the CPU baselines of the path (fp32 compute on
fp16 pages, torch's intra-op threads on the host cores); tests/test_oracle.py
checks them against the numpy oracle, and the GPU tests run them on the
device as the full-size reference of the attention kernels. The product path
(kunserve_amd) never imports this module.

They restate the semantics of oracle.paged_attention_ref:
  decode_attention   its decode_attention (LlamaOp.pforward decode rows,
                     kunserve/worker.py:298-312; pages of
                     kunserve/block_manager.py:786-795; heads
                     kunserve/models.py:55-56): per row, gather its kv_len
                     tokens through the page table, then
                     softmax(q . K^T * sm_scale) . V per query head, query
                     head h reading KV head h // (Hq / Hkv);
  prefill_attention  its prefill_attention (prefill rows,
                     kunserve/request.py:368-391,447-462): the same per row,
                     with q row i of a row of q_len rows seeing positions
                     [0, kv_len - q_len + i];
  copy_blocks        its copy_blocks (LlamaOp.local_copy_blocks,
                     kunserve/worker.py:818-823).
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


def prefill_attention(q: torch.Tensor, q_indptr: np.ndarray, k_pool: torch.Tensor,
                      v_pool: torch.Tensor, layer: int, indptr: np.ndarray,
                      indices: np.ndarray, kv_len: np.ndarray, sm_scale: float,
                      rows=None) -> torch.Tensor:
    """q [T, Hq, D] (rows grouped by q_indptr) and pools [pages, L, Hkv,
    page_size, D] on one device; returns [T, Hq, D] float32 there, causal:
    q row i of row b sees the first kv_len[b] - q_len[b] + i + 1 tokens.
    rows, if given, selects the rows computed (the others stay zero)."""
    T, hq, d = q.shape
    hkv, ps = k_pool.shape[2], k_pool.shape[3]
    g = hq // hkv
    out = torch.zeros((T, hq, d), dtype=torch.float32, device=q.device)
    idx = torch.from_numpy(np.asarray(indices, dtype=np.int64)).to(k_pool.device)
    for b in (range(len(kv_len)) if rows is None else rows):
        q0, q1 = int(q_indptr[b]), int(q_indptr[b + 1])
        n, ql = int(kv_len[b]), q1 - q0
        if ql == 0:
            continue
        pages = idx[int(indptr[b]):int(indptr[b]) + (n + ps - 1) // ps]
        k = k_pool[pages, layer].float().transpose(0, 1).reshape(hkv, -1, d)[:, :n]
        v = v_pool[pages, layer].float().transpose(0, 1).reshape(hkv, -1, d)[:, :n]
        # [ql, Hq, D] -> [Hkv, G * ql, D], query head h = kv head h // G
        qb = q[q0:q1].float().reshape(ql, hkv, g, d).permute(1, 2, 0, 3).reshape(hkv, g * ql, d)
        s = torch.bmm(qb, k.transpose(1, 2).contiguous()) * sm_scale     # [Hkv, G*ql, n]
        last = torch.arange(ql, device=q.device) + (n - ql)               # last visible key
        mask = torch.arange(n, device=q.device)[None, :] > last[:, None]  # [ql, n]
        s.masked_fill_(mask.repeat(g, 1)[None], float("-inf"))
        o = torch.bmm(torch.softmax(s, dim=-1), v.contiguous())           # [Hkv, G*ql, D]
        out[q0:q1] = o.reshape(hkv, g, ql, d).permute(2, 0, 1, 3).reshape(ql, hq, d)
    return out


def copy_blocks(k_pool: torch.Tensor, v_pool: torch.Tensor, src: np.ndarray,
                dst: np.ndarray) -> None:
    """pool[dst[i]] := pool[src[i]] for K and V, whole blocks (all layers)."""
    s = torch.from_numpy(np.asarray(src, dtype=np.int64))
    t = torch.from_numpy(np.asarray(dst, dtype=np.int64))
    for pool in (k_pool, v_pool):
        pool.index_copy_(0, t, pool.index_select(0, s))
