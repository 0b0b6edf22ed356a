"""CPU oracle of the paged-KV attention path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the reference that GPU results are compared
against or as the timed CPU baseline; the product path (kunserve_amd) never
calls it.

The reference's kernels (FlashTransformer, with FlashInfer / flash-attention
underneath) are not present in the reference tree (empty git submodule,
.gitmodules:1-3), so each function restates the semantics fixed by the
reference's Python call sites, in plain numpy (float64 by default):

  decode_attention    LlamaOp.pforward decode rows      kunserve/worker.py:298-312,
                      heads kunserve/models.py:55-56, page size kunserve/models.py:57
  prefill_attention   LlamaOp.pforward prefill rows     kunserve/request.py:368-391,428-462
  append_kv           K/V append into pages             kunserve/block_manager.py:786-795
  rope, rope_append_kv  rotary positions + append (the pforward prologue; positions
                      from the A3 rule, kunserve/request.py:447-462; the rotation itself
                      is inside the absent native LlamaOp, so its pairing convention is
                      taken as a parameter: parity unpinned beyond the closed forms)
  copy_blocks         LlamaOp.local_copy_blocks         kunserve/worker.py:818-823
  swap                swapping_ops.swap                 kunserve/worker.py:646-650,673-681
  kv_pack/kv_scatter  kv_exchange phases 1 and 3        kunserve/flash_backend.py:857-1022
  kv_lens_for_step    first_token_indexes rule          kunserve/request.py:414-462,654-670
  fused_page_ids,     fused / extend page-id space      kunserve/block_manager.py:250-253,
  extend_page_ids,                                      262-269, 755-760
  kept_page_id,
  fused_slab,         which (page, layer) of the pool a fused page uses (same lines;
  fused_pool_copy     the extend layout is a convention, see fused_slab)

Pinning (tests/test_oracle.py): attention is checked against
torch.nn.functional.scaled_dot_product_attention on dense K/V written into
pages by an independent loop, and against closed forms (kv_len 1, q = 0,
page permutation, GQA = repeated-KV MHA, prefill row = decode over its
prefix); block movement is checked bit-exactly against element-wise loops on
pools filled with unique values; kv_lens_for_step against a restated
request lifecycle (also with every row flagged, the use_tensor_cores mode);
the fused map by the invariants the block manager relies on (a kept id
reads its page's bytes in place, fused ids partition the pool's slabs). No
reference golden vectors exist in the reference tree.
"""
from __future__ import annotations

from typing import Sequence

import numpy as np

# ------------------------------------------------------------- page tables


def gather_kv(pool: np.ndarray, layer: int, pages: np.ndarray, kv_len: int) -> np.ndarray:
    """Dense [Hkv, kv_len, D] view of one sequence's K (or V) in `layer`.

    pool is [num_pages, L, Hkv, page_size, D]; token t lives in page
    pages[t // page_size], slot t % page_size (kunserve/block_manager.py:786-795).
    """
    ps = pool.shape[3]
    n = (kv_len + ps - 1) // ps
    blk = pool[np.asarray(pages[:n], dtype=np.int64), layer]        # [n, Hkv, ps, D]
    dense = blk.transpose(1, 0, 2, 3).reshape(pool.shape[2], n * ps, pool.shape[4])
    return dense[:, :kv_len]


def _softmax_rows(s: np.ndarray) -> np.ndarray:
    m = np.max(s, axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    e = np.exp(s - m)
    z = np.sum(e, axis=-1, keepdims=True)
    return e / np.where(z > 0, z, 1.0)


# --------------------------------------------------------------- attention


def decode_attention(q: np.ndarray, k_pool: np.ndarray, v_pool: np.ndarray, layer: int,
                     indptr: np.ndarray, indices: np.ndarray, kv_len: np.ndarray,
                     sm_scale: float, dtype=np.float64) -> np.ndarray:
    """out[b, h] = softmax(q[b, h] . K_b[g(h)]^T * sm_scale) . V_b[g(h)],
    g(h) = h // (Hq // Hkv). q is [B, Hq, D]; returns [B, Hq, D] in `dtype`.
    A row with kv_len 0 yields zeros."""
    B, hq, d = q.shape
    hkv = k_pool.shape[2]
    g = hq // hkv
    out = np.zeros((B, hq, d), dtype=dtype)
    for b in range(B):
        n = int(kv_len[b])
        if n == 0:
            continue
        pages = indices[indptr[b]:indptr[b + 1]]
        K = gather_kv(k_pool, layer, pages, n).astype(dtype)           # [Hkv, n, D]
        V = gather_kv(v_pool, layer, pages, n).astype(dtype)
        qb = q[b].astype(dtype).reshape(hkv, g, d)                     # [Hkv, G, D]
        s = np.matmul(qb, K.transpose(0, 2, 1)) * sm_scale             # [Hkv, G, n]
        out[b] = np.matmul(_softmax_rows(s), V).reshape(hq, d)
    return out


def prefill_attention(q: np.ndarray, q_indptr: np.ndarray, k_pool: np.ndarray,
                      v_pool: np.ndarray, layer: int, indptr: np.ndarray, indices: np.ndarray,
                      kv_len: np.ndarray, sm_scale: float, dtype=np.float64) -> np.ndarray:
    """Causal attention of each row's q_len new tokens (already appended)
    against its kv_len cached tokens: new token i of row b sits at position
    kv_len[b] - q_len[b] + i and sees positions [0, that position]
    (kunserve/request.py:447-462). q is [T, Hq, D]; returns [T, Hq, D]."""
    T, hq, d = q.shape
    hkv = k_pool.shape[2]
    g = hq // hkv
    out = np.zeros((T, hq, d), dtype=dtype)
    for b in range(len(kv_len)):
        q0, q1 = int(q_indptr[b]), int(q_indptr[b + 1])
        ql, n = q1 - q0, int(kv_len[b])
        if ql == 0:
            continue
        pages = indices[indptr[b]:indptr[b + 1]]
        K = gather_kv(k_pool, layer, pages, n).astype(dtype)           # [Hkv, n, D]
        V = gather_kv(v_pool, layer, pages, n).astype(dtype)
        qb = q[q0:q1].astype(dtype).transpose(1, 0, 2).reshape(hkv, g, ql, d)
        s = np.matmul(qb, K[:, None].transpose(0, 1, 3, 2)) * sm_scale  # [Hkv, G, ql, n]
        pos = (n - ql) + np.arange(ql)[:, None]
        s = np.where(np.arange(n)[None, :] <= pos, s, -np.inf)
        o = np.matmul(_softmax_rows(s), V[:, None])                    # [Hkv, G, ql, D]
        out[q0:q1] = o.reshape(hq, ql, d).transpose(1, 0, 2)
    return out


# ---------------------------------------------------------- block movement


def append_kv(k_pool: np.ndarray, v_pool: np.ndarray, layer: int, indptr: np.ndarray,
              indices: np.ndarray, kv_len: np.ndarray, q_indptr: np.ndarray,
              k_new: np.ndarray, v_new: np.ndarray) -> None:
    """In place: new token i of row b (position kv_len[b] - q_len[b] + i)
    goes to page indices[indptr[b] + pos // ps], slot pos % ps."""
    ps = k_pool.shape[3]
    for b in range(len(kv_len)):
        q0, q1 = int(q_indptr[b]), int(q_indptr[b + 1])
        first = int(kv_len[b]) - (q1 - q0)
        for i in range(q1 - q0):
            pos = first + i
            page = int(indices[indptr[b] + pos // ps])
            k_pool[page, layer, :, pos % ps] = k_new[q0 + i]
            v_pool[page, layer, :, pos % ps] = v_new[q0 + i]


def rope(x: np.ndarray, pos: np.ndarray, inv_freq: np.ndarray, interleave: bool) -> np.ndarray:
    """Rotary position embedding of x [T, H, D] at positions pos [T].

    The angle of pair j is the float32 product pos * inv_freq[j] (the rounding
    every fp32 implementation shares); cos, sin and the rotation are then
    evaluated in float64. Pairs are (j, j + D/2) (rotate_half) or, with
    interleave, (2j, 2j + 1). Returns float64."""
    x = np.asarray(x, dtype=np.float64)
    d = x.shape[-1]
    ang = (np.asarray(pos).astype(np.float32)[:, None] * np.asarray(inv_freq, np.float32)[None, :])
    c = np.cos(ang.astype(np.float64))[:, None, :]
    s = np.sin(ang.astype(np.float64))[:, None, :]
    if interleave:
        a, b = x[..., 0::2], x[..., 1::2]
        out = np.empty_like(x)
        out[..., 0::2] = a * c - b * s
        out[..., 1::2] = b * c + a * s
        return out
    a, b = x[..., : d // 2], x[..., d // 2:]
    return np.concatenate([a * c - b * s, b * c + a * s], axis=-1)


def token_positions(kv_len: np.ndarray, q_indptr: np.ndarray) -> np.ndarray:
    """Position of every new token: row b's token i sits at kv_len[b] - q_len[b] + i
    (kunserve/request.py:447-462)."""
    out = []
    for b in range(len(kv_len)):
        q0, q1 = int(q_indptr[b]), int(q_indptr[b + 1])
        out.extend(range(int(kv_len[b]) - (q1 - q0), int(kv_len[b])))
    return np.asarray(out, dtype=np.int64)


def rope_append_kv(k_pool: np.ndarray, v_pool: np.ndarray, layer: int, indptr: np.ndarray,
                   indices: np.ndarray, kv_len: np.ndarray, q_indptr: np.ndarray,
                   q: np.ndarray, k_new: np.ndarray, v_new: np.ndarray,
                   inv_freq: np.ndarray, interleave: bool) -> np.ndarray:
    """The attention prologue of a step: rotate q and the new k at their token
    positions, append the rotated k and v into the pages (in place). Returns
    the rotated q, rounded to the pool dtype."""
    pos = token_positions(kv_len, q_indptr)
    q_rot = rope(q, pos, inv_freq, interleave).astype(k_pool.dtype)
    k_rot = rope(k_new, pos, inv_freq, interleave).astype(k_pool.dtype)
    append_kv(k_pool, v_pool, layer, indptr, indices, kv_len, q_indptr, k_rot, v_new)
    return q_rot


def copy_blocks(pool: np.ndarray, src: Sequence[int], dst: Sequence[int]) -> None:
    """In place: pool[dst[i]] := pool[src[i]] (whole block, all layers)."""
    snap = pool[np.asarray(src, dtype=np.int64)].copy()
    pool[np.asarray(dst, dtype=np.int64)] = snap


def swap(src: Sequence[int], dst: Sequence[int], from_pool: np.ndarray,
         to_pool: np.ndarray) -> None:
    """In place: to_pool[dst[i]] := from_pool[src[i]] (kunserve/worker.py:646-650)."""
    for s, t in zip(src, dst):
        to_pool[int(t)] = from_pool[int(s)]


def kv_pack(k_pool: np.ndarray, v_pool: np.ndarray, layer_begin: int, layer_end: int,
            page_ids: Sequence[int]) -> np.ndarray:
    """Scratch [layers][n][2 (K, V)][Hkv][page_size][D] of the given pages."""
    ids = np.asarray(page_ids, dtype=np.int64)
    k = k_pool[ids, layer_begin:layer_end]          # [n, l, Hkv, ps, D]
    v = v_pool[ids, layer_begin:layer_end]
    return np.stack([k, v], axis=2).transpose(1, 0, 2, 3, 4, 5).copy()


def kv_scatter(k_pool: np.ndarray, v_pool: np.ndarray, layer_begin: int, layer_end: int,
               page_ids: Sequence[int], scratch: np.ndarray) -> None:
    """In place: inverse of kv_pack."""
    ids = np.asarray(page_ids, dtype=np.int64)
    s = scratch.transpose(1, 0, 2, 3, 4, 5)         # [n, l, 2, Hkv, ps, D]
    k_pool[ids, layer_begin:layer_end] = s[:, :, 0]
    v_pool[ids, layer_begin:layer_end] = s[:, :, 1]


# ------------------------------------------------------ host conventions


def kv_lens_for_step(first_token_indexes: Sequence[int], q_lens: Sequence[int],
                     is_prefill_requests: Sequence[int], use_tensor_cores: bool = False,
                     is_context_stage: Sequence[int] | None = None,
                     pages_per_row: Sequence[int] | None = None,
                     page_size: int = 0) -> np.ndarray:
    """kv_len after append. Prefill rows: first = prefill_begin_index, so
    first + q_len; decode rows: first = prompt_len + output_len, which
    already counts the token being decoded (kunserve/request.py:414-462).
    With use_tensor_cores every row is flagged prefill
    (kunserve/request.py:667-670). is_context_stage, when given, is each
    row's real stage and decides. Otherwise a one-token row past position 0
    is a decode row only when its table cannot hold position `first` (a
    prefill chunk's table holds ceil((first + 1) / page_size) pages,
    kunserve/block_manager.py:786-795); when it can, the row is ambiguous
    and ValueError is raised."""
    out = []
    for b, (f, ql, flag) in enumerate(zip(first_token_indexes, q_lens, is_prefill_requests)):
        if is_context_stage is not None:
            decode = not is_context_stage[b]
        elif use_tensor_cores and flag and ql == 1 and f > 0:
            if pages_per_row is None or pages_per_row[b] * page_size > f:
                raise ValueError(f"row {b}: one-token row at {f} is ambiguous under "
                                 f"use_tensor_cores")
            decode = True
        else:
            decode = not flag
        out.append(f if decode else f + ql)
    return np.asarray(out, dtype=np.int64)


def fused_page_ids(base_page: int, num_base_pages: int, num_instances: int) -> list[int]:
    """convert_to_pipeline_format: pre-fusion page b of an instance with P
    base pages becomes fused ids {i * P + b} (kunserve/block_manager.py:250-253)."""
    return [num_base_pages * i + base_page for i in range(num_instances)]


def extend_page_ids(num_base_pages_fused: int, num_extend: int) -> list[int]:
    """add_ex_fusion_blocks: extend pages follow the fused base region
    (kunserve/block_manager.py:262-269)."""
    return [num_base_pages_fused + k for k in range(num_extend)]


def kept_page_id(base_page: int, num_base_pages_fused: int, fusion_size: int,
                 fusion_rank: int) -> int:
    """free_blocks_into_fusion_except: a stale request keeps fused id
    (P_fused // fusion_size) * rank + b (kunserve/block_manager.py:755-760)."""
    return num_base_pages_fused // fusion_size * fusion_rank + base_page


def fused_slab(fused_id: int, local_layer: int, base_pages: int, fusion_size: int,
               num_layers: int) -> tuple[int, int]:
    """(page, layer) of the unfused [pages, num_layers, ...] pool that fused
    page `fused_id` uses for layer `local_layer` of its stage.

    Base ids (< P * N): convert_to_pipeline_format splits free page b into
    fused ids i * P + b (kunserve/block_manager.py:250-253), one per stage of
    G = num_layers / N layers, and a stale request of rank r keeps r * P + b
    with its KV still in place (kunserve/block_manager.py:755-760): fused
    id i * P + b is layers [i * G, (i + 1) * G) of page b. Extend ids
    (>= P * N, kunserve/block_manager.py:262-269) are G-layer pages carved
    from the pages behind the base ones (the dropped weight memory), N per
    page, in order: that layout is inside the absent native LlamaOp, so it
    is this build's convention, pinned only by the invariants the tests
    check (disjoint from the base pages, every slab used once)."""
    g = num_layers // fusion_size
    if fused_id < base_pages * fusion_size:
        return fused_id % base_pages, (fused_id // base_pages) * g + local_layer
    e = fused_id - base_pages * fusion_size
    return base_pages + e // fusion_size, (e % fusion_size) * g + local_layer


def fused_pool_copy(pool: np.ndarray, base_pages: int, fusion_size: int) -> np.ndarray:
    """The pool as the fused id space sees it: [P*N + E, G, Hkv, ps, D], slab
    by slab through fused_slab (an element loop over pages and layers)."""
    pages, layers = pool.shape[:2]
    g = layers // fusion_size
    out = np.empty((pages * fusion_size, g) + pool.shape[2:], dtype=pool.dtype)
    for f in range(pages * fusion_size):
        for j in range(g):
            out[f, j] = pool[fused_slab(f, j, base_pages, fusion_size, layers)]
    return out
