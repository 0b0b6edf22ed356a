"""Shared helpers of the GPU parity tests (test code only)."""
from __future__ import annotations

import math

import numpy as np
import torch

from kunserve_amd import KVPool, PageTable

ATOL = 2e-3   # max-abs tolerance for fp16 attention outputs, fp32 accumulation
# bf16 keeps 8 significant bits to fp16's 11: the same bound scaled by 2^3,
# rounded up (output rounding alone is up to 2^-9 |o|, and P enters the
# P.V product as bf16).
ATOL_BF16 = 2e-2
# The same in relative form, over a whole output: rounding the output to
# bf16 (unit roundoff 2^-9) and the probabilities to bf16 before P.V (2^-9 of
# each term, uncorrelated, so about 2^-9 of the row sum again) give an RMS
# relative error of about 2 * 2^-9 / sqrt(3) = 1.1e-3; 8e-3 leaves a margin
# of 7 and still fails a term dropped or doubled in a row of 100 keys.
RTOL_BF16 = 8e-3


def random_pool(num_pages, num_layers, num_kv_heads, page_size, head_dim, device, seed,
                scale=1.0, dtype=torch.float16) -> KVPool:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    pool = KVPool.allocate(num_pages, num_layers, num_kv_heads, page_size, head_dim, device,
                           dtype)
    for t in (pool.k, pool.v):
        # fill layer by layer to bound the temporary fp32 buffer
        for layer in range(num_layers):
            t[:, layer].copy_((torch.randn(t[:, layer].shape, generator=g, device=device,
                                           dtype=torch.float32) * scale).to(dtype))
    return pool


def random_tensor(shape, device, seed, scale=1.0, dtype=torch.float16) -> torch.Tensor:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return (torch.randn(shape, generator=g, device=device) * scale).to(dtype)


def to_numpy(t: torch.Tensor) -> np.ndarray:
    """Host copy; bf16 (which numpy lacks) becomes float32, exactly."""
    t = t.cpu()
    return t.float().numpy() if t.dtype == torch.bfloat16 else t.numpy()


def compact_for_oracle(pool: KVPool, layer: int, indptr: np.ndarray, indices: np.ndarray,
                       rows=None):
    """Host copies of only the pages the selected rows use (one layer), with
    the table renumbered into the compact pool: keeps oracle inputs small
    when the device pool is many GiB."""
    rows = np.arange(len(indptr) - 1) if rows is None else np.asarray(rows)
    pages = [indices[indptr[b]:indptr[b + 1]] for b in rows]
    used = np.concatenate(pages) if pages else np.zeros(0, np.int64)
    uniq, inv = np.unique(used, return_inverse=True)
    sel = torch.from_numpy(uniq.astype(np.int64)).to(pool.device)
    k = to_numpy(pool.k[:, layer].index_select(0, sel)[:, None])
    v = to_numpy(pool.v[:, layer].index_select(0, sel)[:, None])
    new_indptr = np.zeros(len(rows) + 1, dtype=np.int64)
    np.cumsum([len(p) for p in pages], out=new_indptr[1:])
    return k, v, new_indptr, inv.astype(np.int64)


def torch_decode_ref(pool: KVPool, layer: int, indptr, indices, kv_len, q: torch.Tensor,
                     sm_scale: float | None = None) -> torch.Tensor:
    """Decode attention of every row in fp32 on the pool's device, by the
    PyTorch restatement of the oracle (oracle.torch_cpu, pinned against the
    numpy oracle on the CPU): the full-size reference of the decode tests."""
    from oracle import torch_cpu

    scale = 1.0 / math.sqrt(pool.head_dim) if sm_scale is None else sm_scale
    return torch_cpu.decode_attention(q, pool.k, pool.v, 0 if pool.num_layers == 1 else layer,
                                      np.asarray(indptr), np.asarray(indices),
                                      np.asarray(kv_len), scale)


def table_from_csr(indptr, indices, kv_len, device) -> PageTable:
    return PageTable(np.asarray(indptr, np.int32), np.asarray(indices, np.int32),
                     np.asarray(kv_len, np.int32), device)


def rel_err(a, b) -> float:
    """||a - b|| / ||b|| over the whole arrays (Frobenius), in float64."""
    a = a.float().cpu().numpy() if isinstance(a, torch.Tensor) else np.asarray(a)
    b = b.float().cpu().numpy() if isinstance(b, torch.Tensor) else np.asarray(b)
    a, b = a.astype(np.float64), b.astype(np.float64)
    nb = float(np.linalg.norm(b))
    return float(np.linalg.norm(a - b)) / nb if nb else float(np.linalg.norm(a))


def max_abs(a, b) -> float:
    a = a.float().cpu().numpy() if isinstance(a, torch.Tensor) else np.asarray(a)
    b = b.float().cpu().numpy() if isinstance(b, torch.Tensor) else np.asarray(b)
    return float(np.max(np.abs(a.astype(np.float64) - b.astype(np.float64)))) if a.size else 0.0
