"""Host side of the paged-KV path: pool, page tables, plans and op wrappers.

PyTorch supplies device memory and the current stream; every byte of device
work goes through libkunserve_hip.so (include/kunserve_hip.h). There is no
CPU or PyTorch fallback: without the library each op raises.

Reference contracts restated here:
  * KV pool [num_blocks, num_layers, num_kv_heads, block_size, head_dim],
    K and V separate (kunserve/worker.py:168-176); block bytes
    2 * L * Hkv * bs * D * dtype (kunserve/worker.py:205-218).
  * Ragged block tables List[List[int]] (kunserve/block_manager.py:786-795):
    token t of a request lives in page table[t // bs], slot t % bs.
  * Per-step arguments of LlamaOp.pforward (kunserve/worker.py:270-312,
    kunserve/request.py:414-462,654-670).
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np
import torch

from . import _lib

FP16 = torch.float16


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _i32(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.int32))


_DTYPES = {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16}


class KVPool:
    """Separate K and V pools of shape [num_pages, num_layers, num_kv_heads,
    page_size, head_dim] (any strides with head_dim contiguous), float16 or
    bfloat16 (the reference's --dtype, kunserve/kunserve_config.py:61); q,
    outputs and new K/V passed with a pool must have its dtype."""

    def __init__(self, k: torch.Tensor, v: torch.Tensor, owner=None):
        """owner: the PmmPool whose memory k and v view, if any; the view
        stops being usable once that pool's pages are remapped."""
        if k.shape != v.shape or k.stride() != v.stride() or k.dim() != 5:
            raise ValueError("K and V pools must be 5-D with identical shape and strides")
        if k.dtype != v.dtype or k.dtype not in _DTYPES:
            raise ValueError("KV pools must both be float16 or both bfloat16")
        if k.stride(-1) != 1:
            raise ValueError("head_dim must be contiguous")
        self.k, self.v = k, v
        self.dtype = k.dtype
        self.num_pages, self.num_layers, self.num_kv_heads, self.page_size, self.head_dim = k.shape
        self._desc = _lib.KVPool(
            k.data_ptr(), v.data_ptr(), self.num_pages, k.stride(0), k.stride(1), k.stride(2),
            k.stride(3), self.num_layers, self.num_kv_heads, self.page_size, self.head_dim,
            _DTYPES[k.dtype],
        )
        self._owner = owner
        self._generation = owner.generation if owner is not None else 0

    @classmethod
    def allocate(cls, num_pages: int, num_layers: int, num_kv_heads: int, page_size: int,
                 head_dim: int, device="cuda", dtype: torch.dtype = FP16) -> "KVPool":
        shape = (num_pages, num_layers, num_kv_heads, page_size, head_dim)
        return cls(torch.empty(shape, dtype=dtype, device=device),
                   torch.empty(shape, dtype=dtype, device=device))

    def check_dtype(self, *tensors: torch.Tensor) -> None:
        for t in tensors:
            if t is not None and t.dtype != self.dtype:
                raise ValueError(f"tensor dtype {t.dtype} does not match the pool's {self.dtype}")

    @property
    def device(self) -> torch.device:
        return self.k.device

    @property
    def block_bytes(self) -> int:
        """Bytes of one block of K plus V over all layers (worker.py:205-218)."""
        return 2 * self.num_layers * self.num_kv_heads * self.page_size * self.head_dim * 2

    def desc(self) -> ctypes.pointer:
        if self._owner is not None and self._owner.generation != self._generation:
            raise RuntimeError("this KVPool predates a pmm drop or restore of its pages; "
                               "use the owner's current pool")
        return ctypes.byref(self._desc)


# ------------------------------------------------------------ step arguments


def kv_lens_for_step(first_token_indexes: Sequence[int], q_lens: Sequence[int],
                     is_prefill_requests: Sequence[int]) -> np.ndarray:
    """KV length of each row after this step's tokens are appended.

    kunserve/request.py:447-462: a prefill row's first index is
    prefill_begin_index (tokens already cached), so kv_len = first + q_len;
    a decode row's first index is prompt_len + output_len, which already
    counts the token being decoded (the block allocation of
    kunserve/request.py:414-423 uses the same count), so kv_len = first.
    In both cases the new tokens occupy positions [kv_len - q_len, kv_len).
    """
    first = np.asarray(first_token_indexes, dtype=np.int64)
    ql = np.asarray(q_lens, dtype=np.int64)
    flag = np.asarray(is_prefill_requests, dtype=np.int64)
    if not (first.shape == ql.shape == flag.shape):
        raise ValueError("first_token_indexes, q_lens and is_prefill_requests differ in length")
    kv = np.where(flag != 0, first + ql, first)
    if np.any(kv < ql):
        bad = int(np.argmax(kv < ql))
        raise ValueError(f"row {bad}: kv_len {kv[bad]} shorter than its {ql[bad]} new tokens")
    return kv.astype(np.int32)


def csr_from_lists(pages_of_reqs: Sequence[Sequence[int]], kv_len: np.ndarray,
                   page_size: int, num_pages: int) -> tuple[np.ndarray, np.ndarray]:
    """Ragged page lists -> (indptr, indices) int32, validated.

    Each row must hold at least ceil(kv_len / page_size) pages
    (kunserve/block_manager.py:493-500,786-795); only those are kept.
    """
    n = len(pages_of_reqs)
    if len(kv_len) != n:
        raise ValueError(f"{n} page lists but {len(kv_len)} kv lengths")
    need = (np.asarray(kv_len, dtype=np.int64) + page_size - 1) // page_size
    indptr = np.zeros(n + 1, dtype=np.int64)
    np.cumsum(need, out=indptr[1:])
    indices = np.empty(int(indptr[-1]), dtype=np.int64)
    for b, pages in enumerate(pages_of_reqs):
        k = int(need[b])
        if len(pages) < k:
            raise ValueError(f"row {b}: {len(pages)} pages for {int(kv_len[b])} tokens "
                             f"(page_size {page_size}) needs {k}")
        indices[indptr[b]:indptr[b + 1]] = pages[:k]
    if indices.size and (indices.min() < 0 or indices.max() >= num_pages):
        bad = int(indices[(indices < 0) | (indices >= num_pages)][0])
        raise IndexError(f"page id {bad} outside the pool [0, {num_pages})")
    return indptr.astype(np.int32), indices.astype(np.int32)


class PageTable:
    """Per-step CSR page table, on the device and mirrored on the host."""

    def __init__(self, indptr: np.ndarray, indices: np.ndarray, kv_len: np.ndarray,
                 device: torch.device):
        self.indptr_host = _i32(indptr)
        self.indices_host = _i32(indices)
        self.kv_len_host = _i32(kv_len)
        self.num_seqs = len(self.kv_len_host)
        if len(self.indptr_host) != self.num_seqs + 1:
            raise ValueError("indptr must have num_seqs + 1 entries")
        # One upload for the three arrays.
        packed = np.concatenate([self.indptr_host, self.kv_len_host, self.indices_host])
        dev = torch.from_numpy(packed).to(device, non_blocking=False)
        n = self.num_seqs
        self.indptr = dev[: n + 1]
        self.kv_len = dev[n + 1: 2 * n + 1]
        self.indices = dev[2 * n + 1:]
        self._storage = dev
        self._desc = _lib.PageTable(self.indptr.data_ptr(), self.indices.data_ptr(),
                                    self.kv_len.data_ptr(), n)

    @classmethod
    def from_lists(cls, pages_of_reqs: Sequence[Sequence[int]], kv_len, pool: KVPool
                   ) -> "PageTable":
        kv = _i32(kv_len)
        indptr, indices = csr_from_lists(pages_of_reqs, kv, pool.page_size, pool.num_pages)
        return cls(indptr, indices, kv, pool.device)

    def desc(self):
        return ctypes.byref(self._desc)


def _tensor3(t: torch.Tensor) -> _lib.Tensor3:
    if t.dim() != 3 or t.stride(-1) != 1:
        raise ValueError("expected a [tokens, heads, head_dim] tensor with head_dim contiguous")
    if t.dtype not in _DTYPES:
        raise ValueError("expected float16 or bfloat16")
    return _lib.Tensor3(t.data_ptr(), t.stride(0), t.stride(1))


def _num_cus(device: torch.device) -> int:
    return torch.cuda.get_device_properties(device).multi_processor_count


class DecodePlan:
    """Partitioning of decode rows, computed on the host once per step and
    shared by every layer (kunserve_decode_plan)."""

    def __init__(self, kv_len_host: Sequence[int], num_qo_heads: int, num_kv_heads: int,
                 device: torch.device, part_tokens: int = 0, num_cus: Optional[int] = None):
        kv = _i32(kv_len_host)
        n = len(kv)
        cap = _lib.lib().kunserve_decode_plan_bound(kv.ctypes.data if n else None, n)
        buf = np.zeros(max(int(cap), 4), dtype=np.int32)
        self.info = _lib.DecodePlanInfo()
        cus = num_cus if num_cus is not None else _num_cus(device)
        _lib.call("kunserve_decode_plan", kv.ctypes.data if n else None, n, num_qo_heads,
                  num_kv_heads, cus, part_tokens, buf.ctypes.data, buf.size,
                  ctypes.byref(self.info))
        self.plan_host = buf[: self.info.plan_ints].copy()
        self.plan = torch.from_numpy(self.plan_host).to(device) if self.info.plan_ints else None
        self.num_qo_heads = num_qo_heads
        self.num_kv_heads = num_kv_heads

    def workspace_bytes(self, head_dim: int) -> int:
        return int(_lib.lib().kunserve_decode_workspace_bytes(
            ctypes.byref(self.info), self.num_qo_heads, head_dim))


class PrefillPlan:
    """(row, q tile, q head) work items of the prefill rows, XCD-ordered
    (kunserve_prefill_plan). Steps with too few items to fill the device
    split each item's KV range; the merge runs inside paged_prefill."""

    def __init__(self, q_indptr_host: Sequence[int], kv_len_host: Sequence[int],
                 num_qo_heads: int, num_kv_heads: int, device: torch.device,
                 num_cus: Optional[int] = None):
        qi = _i32(q_indptr_host)
        kv = _i32(kv_len_host)
        n = len(kv)
        if len(qi) != n + 1:
            raise ValueError("q_indptr must have num_seqs + 1 entries")
        cap = int(_lib.lib().kunserve_prefill_plan_bound(qi.ctypes.data, n, num_qo_heads))
        buf = np.zeros(max(cap, 3), dtype=np.int32)
        self.info = _lib.PrefillPlanInfo()
        cus = num_cus if num_cus is not None else _num_cus(device)
        _lib.call("kunserve_prefill_plan", qi.ctypes.data, kv.ctypes.data if n else None, n,
                  num_qo_heads, num_kv_heads, cus, buf.ctypes.data, buf.size,
                  ctypes.byref(self.info))
        self.plan_host = buf[: self.info.plan_ints].copy()
        self.plan = torch.from_numpy(self.plan_host).to(device) if self.info.plan_ints else None

    def workspace_bytes(self) -> int:
        return int(_lib.lib().kunserve_prefill_workspace_bytes(ctypes.byref(self.info)))


# ------------------------------------------------------------------ ops


def copy_blocks(pool: KVPool, src_ids, dst_ids) -> None:
    """pool[dst_ids[i]] := pool[src_ids[i]] for K and V, every layer
    (LlamaOp.local_copy_blocks, kunserve/worker.py:818-823)."""
    src = _ids_on_device(src_ids, pool)
    dst = _ids_on_device(dst_ids, pool)
    if src.numel() != dst.numel():
        raise ValueError("src and dst id lists differ in length")
    if src.numel() == 0:
        return
    _lib.call("kunserve_copy_blocks", pool.desc(), src.data_ptr(), dst.data_ptr(), src.numel(),
              _stream_ptr(pool.device))


def _ids_on_device(ids, pool: KVPool) -> torch.Tensor:
    if isinstance(ids, torch.Tensor) and ids.is_cuda:
        if ids.dtype != torch.int32:
            raise ValueError("device id tensors must be int32")
        return ids.contiguous()
    arr = np.asarray(ids, dtype=np.int64).reshape(-1)
    if arr.size and (arr.min() < 0 or arr.max() >= pool.num_pages):
        raise IndexError(f"block id outside the pool [0, {pool.num_pages})")
    return torch.from_numpy(arr.astype(np.int32)).to(pool.device)


def kv_pack(pool: KVPool, layer_begin: int, layer_end: int, page_ids,
            scratch: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Gathers layers [layer_begin, layer_end) of page_ids into a contiguous
    scratch buffer [layers][n][K|V][heads][page_size][head_dim]
    (kv_exchange phase 1, kunserve/flash_backend.py:930-985)."""
    ids = _ids_on_device(page_ids, pool)
    n = ids.numel()
    nbytes = int(_lib.lib().kunserve_kv_pack_bytes(pool.desc(), layer_end - layer_begin, n))
    if scratch is None:
        scratch = torch.empty(max(nbytes // 2, 1), dtype=pool.dtype, device=pool.device)
    _lib.call("kunserve_kv_pack", pool.desc(), layer_begin, layer_end, ids.data_ptr(), n,
              scratch.data_ptr(), scratch.numel() * scratch.element_size(),
              _stream_ptr(pool.device))
    return scratch


def kv_scatter(pool: KVPool, layer_begin: int, layer_end: int, page_ids,
               scratch: torch.Tensor) -> None:
    """Inverse of kv_pack: writes the scratch layout into page_ids
    (kv_exchange phase 3)."""
    ids = _ids_on_device(page_ids, pool)
    _lib.call("kunserve_kv_scatter", pool.desc(), layer_begin, layer_end, ids.data_ptr(),
              ids.numel(), scratch.data_ptr(), scratch.numel() * scratch.element_size(),
              _stream_ptr(pool.device))


def swap(source_block_ids: Sequence[int], target_block_ids: Sequence[int], is_swap_in: bool,
         k_cache: torch.Tensor, v_cache: torch.Tensor, k_swap: torch.Tensor,
         v_swap: torch.Tensor) -> None:
    """torch.ops.swapping_ops.swap (kunserve/worker.py:646-650,673-681).

    is_swap_in: CPU block source_block_ids[i] -> GPU block target_block_ids[i];
    otherwise GPU -> CPU. Enqueued on the current stream of k_cache's device,
    without synchronising. k_swap / v_swap must be pinned host tensors.
    """
    if len(source_block_ids) != len(target_block_ids):
        raise ValueError("source and target block lists differ in length")
    for t in (k_cache, v_cache):
        if not t.is_cuda or not t.is_contiguous():
            raise ValueError("k_cache / v_cache must be contiguous device tensors")
    for t in (k_swap, v_swap):
        if t.is_cuda or not t.is_pinned() or not t.is_contiguous():
            raise ValueError("k_swap / v_swap must be contiguous pinned host tensors")
    if k_cache.shape[1:] != k_swap.shape[1:] or k_cache.dtype != k_swap.dtype:
        raise ValueError("cache and swap blocks differ in shape or dtype")
    n = len(source_block_ids)
    if n == 0:
        return
    src = np.ascontiguousarray(np.asarray(source_block_ids, dtype=np.int64))
    dst = np.ascontiguousarray(np.asarray(target_block_ids, dtype=np.int64))
    block_bytes = k_cache[0].numel() * k_cache.element_size()
    _lib.call("kunserve_swap_blocks", src.ctypes.data, dst.ctypes.data, n, int(bool(is_swap_in)),
              k_cache.data_ptr(), v_cache.data_ptr(), k_cache.shape[0], k_swap.data_ptr(),
              v_swap.data_ptr(), k_swap.shape[0], block_bytes, _stream_ptr(k_cache.device))


def append_kv(pool: KVPool, layer: int, table: PageTable, q_indptr: torch.Tensor,
              k_new: torch.Tensor, v_new: torch.Tensor) -> None:
    """Writes the new tokens' K/V rows into their pages for one layer."""
    if k_new.shape != v_new.shape or k_new.shape[1:] != (pool.num_kv_heads, pool.head_dim):
        raise ValueError(f"k_new / v_new must be [tokens, {pool.num_kv_heads}, {pool.head_dim}]")
    if q_indptr.numel() != table.num_seqs + 1:
        raise ValueError("q_indptr must have num_seqs + 1 entries")
    pool.check_dtype(k_new, v_new)
    kd, vd = _tensor3(k_new), _tensor3(v_new)
    _lib.call("kunserve_append_kv", pool.desc(), layer, table.desc(), q_indptr.data_ptr(),
              k_new.shape[0], ctypes.byref(kd), ctypes.byref(vd), _stream_ptr(pool.device))


def rope_inv_freq(head_dim: int, theta: float = 10000.0,
                  device: Optional[torch.device] = None) -> torch.Tensor:
    """Llama rotary frequencies theta^(-2j / head_dim), j < head_dim / 2, in
    float32 (the table kunserve_rope_append_kv takes)."""
    inv = 1.0 / (np.float32(theta) ** (np.arange(0, head_dim, 2, dtype=np.float32)
                                       / np.float32(head_dim)))
    t = torch.from_numpy(inv.astype(np.float32))
    return t.to(device) if device is not None else t


def rope_append_kv(pool: KVPool, layer: int, table: PageTable, q_indptr: torch.Tensor,
                   q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                   inv_freq: torch.Tensor, interleave: bool = False) -> torch.Tensor:
    """The attention prologue of one layer: rotates q in place and k_new at
    each new token's position, and writes the rotated k and v_new into their
    pages. Returns q."""
    if k_new.shape != v_new.shape or k_new.shape[1:] != (pool.num_kv_heads, pool.head_dim):
        raise ValueError(f"k_new / v_new must be [tokens, {pool.num_kv_heads}, {pool.head_dim}]")
    if q.shape[0] != k_new.shape[0] or q.shape[2] != pool.head_dim:
        raise ValueError(f"q {tuple(q.shape)} does not match k_new {tuple(k_new.shape)}")
    if q_indptr.numel() != table.num_seqs + 1:
        raise ValueError("q_indptr must have num_seqs + 1 entries")
    if (inv_freq.dtype != torch.float32 or inv_freq.numel() != pool.head_dim // 2
            or inv_freq.device != q.device):
        raise ValueError(f"inv_freq must be {pool.head_dim // 2} float32 values on {q.device}")
    inv_freq = inv_freq.contiguous()
    pool.check_dtype(q, k_new, v_new)
    qd, kd, vd = _tensor3(q), _tensor3(k_new), _tensor3(v_new)
    _lib.call("kunserve_rope_append_kv", pool.desc(), layer, table.desc(), q_indptr.data_ptr(),
              k_new.shape[0], ctypes.byref(qd), q.shape[1], ctypes.byref(kd), ctypes.byref(vd),
              inv_freq.data_ptr(), int(bool(interleave)), _stream_ptr(pool.device))
    return q


def paged_decode(pool: KVPool, layer: int, table: PageTable, q: torch.Tensor, plan: DecodePlan,
                 sm_scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
                 workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Decode attention of q [num_seqs, Hq, D] over each row's pages."""
    hq = q.shape[1]
    if q.shape[0] != table.num_seqs or q.shape[2] != pool.head_dim:
        raise ValueError(f"q shape {tuple(q.shape)} does not match {table.num_seqs} rows, "
                         f"head_dim {pool.head_dim}")
    if out is None:
        out = torch.empty_like(q)
    pool.check_dtype(q, out)
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(pool.head_dim)
    need = plan.workspace_bytes(pool.head_dim)
    if need > 0 and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=pool.device)
    qd, od = _tensor3(q), _tensor3(out)
    _lib.call("kunserve_paged_decode", pool.desc(), layer, table.desc(), ctypes.byref(qd),
              ctypes.byref(od), hq, ctypes.c_float(scale),
              _ptr(plan.plan), ctypes.byref(plan.info), _ptr(workspace),
              0 if workspace is None else workspace.numel() * workspace.element_size(),
              _stream_ptr(pool.device))
    return out


def paged_prefill(pool: KVPool, layer: int, table: PageTable, q_indptr: torch.Tensor,
                  q: torch.Tensor, plan: PrefillPlan, sm_scale: Optional[float] = None,
                  out: Optional[torch.Tensor] = None,
                  workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Causal chunked-prefill attention of ragged q [num_tokens, Hq, D]."""
    if out is None:
        out = torch.empty_like(q)
    pool.check_dtype(q, out)
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(pool.head_dim)
    need = plan.workspace_bytes()
    if need > 0 and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=pool.device)
    qd, od = _tensor3(q), _tensor3(out)
    _lib.call("kunserve_paged_prefill", pool.desc(), layer, table.desc(), q_indptr.data_ptr(),
              ctypes.byref(qd), ctypes.byref(od), q.shape[1], ctypes.c_float(scale),
              _ptr(plan.plan), ctypes.byref(plan.info), _ptr(workspace),
              0 if workspace is None else workspace.numel() * workspace.element_size(),
              _stream_ptr(pool.device))
    return out


@dataclass
class _Subset:
    rows: np.ndarray            # row indices into the batch
    tokens: Optional[torch.Tensor]  # token indices into q (None: all tokens, in order)
    table: PageTable
    q_indptr: Optional[torch.Tensor]
    plan: object


class AttentionStep:
    """The attention stage of one LlamaOp.pforward step, prepared once from
    the step's host arguments and run for every layer.

    Per layer: append the new K/V of every row, then decode attention for
    decode rows (q_len == 1, flag 0) and causal chunked-prefill attention for
    prefill rows (flag 1; with use_tensor_cores every row is flagged,
    kunserve/request.py:667-670).
    """

    def __init__(self, pool: KVPool, num_qo_heads: int, q_lens: Sequence[int],
                 first_token_indexes: Sequence[int], is_prefill_requests: Sequence[int],
                 pages_of_reqs: Sequence[Sequence[int]], sm_scale: Optional[float] = None,
                 decode_part_tokens: int = 0):
        self.pool = pool
        self.num_qo_heads = num_qo_heads
        dev = pool.device
        q_lens = np.asarray(q_lens, dtype=np.int64)
        flags = np.asarray(is_prefill_requests, dtype=np.int64)
        if np.any(q_lens < 1):
            raise ValueError("every row needs at least one input token")
        if np.any((flags == 0) & (q_lens != 1)):
            raise ValueError("decode rows (flag 0) must have exactly one input token")
        self.kv_len = kv_lens_for_step(first_token_indexes, q_lens, flags)
        self.q_indptr_host = np.zeros(len(q_lens) + 1, dtype=np.int32)
        np.cumsum(q_lens, out=self.q_indptr_host[1:])
        self.num_tokens = int(self.q_indptr_host[-1])
        self.table = PageTable.from_lists(pages_of_reqs, self.kv_len, pool)
        self.q_indptr = torch.from_numpy(self.q_indptr_host).to(dev)
        self.scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(pool.head_dim)

        self.decode = self.prefill = None
        all_rows = np.arange(len(q_lens))
        dec_rows = all_rows[flags == 0]
        pre_rows = all_rows[flags != 0]
        if dec_rows.size:
            sub_pages = [pages_of_reqs[i] for i in dec_rows]
            table = (self.table if dec_rows.size == len(q_lens)
                     else PageTable.from_lists(sub_pages, self.kv_len[dec_rows], pool))
            tokens = (None if dec_rows.size == len(q_lens)
                      else torch.from_numpy(self.q_indptr_host[dec_rows].astype(np.int64)).to(dev))
            plan = DecodePlan(self.kv_len[dec_rows], num_qo_heads, pool.num_kv_heads, dev,
                              part_tokens=decode_part_tokens)
            self.decode = _Subset(dec_rows, tokens, table, None, plan)
        if pre_rows.size:
            if pre_rows.size == len(q_lens):
                table, tokens, qi = self.table, None, self.q_indptr_host
            else:
                table = PageTable.from_lists([pages_of_reqs[i] for i in pre_rows],
                                             self.kv_len[pre_rows], pool)
                tok = np.concatenate([np.arange(self.q_indptr_host[i], self.q_indptr_host[i + 1])
                                      for i in pre_rows])
                tokens = torch.from_numpy(tok.astype(np.int64)).to(dev)
                qi = np.zeros(pre_rows.size + 1, dtype=np.int32)
                np.cumsum(q_lens[pre_rows], out=qi[1:])
            plan = PrefillPlan(qi, self.kv_len[pre_rows], num_qo_heads, pool.num_kv_heads, dev)
            self.prefill = _Subset(pre_rows, tokens, table, torch.from_numpy(qi).to(dev), plan)
        # Scratch shared by every layer of the step (launches are serialised on one stream).
        ws = max(self.decode.plan.workspace_bytes(pool.head_dim) if self.decode else 0,
                 self.prefill.plan.workspace_bytes() if self.prefill else 0)
        self.workspace = torch.empty(ws, dtype=torch.uint8, device=dev) if ws > 0 else None

    def run(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
            out: Optional[torch.Tensor] = None,
            rope: Optional[tuple] = None) -> torch.Tensor:
        """q [num_tokens, Hq, D], k/v [num_tokens, Hkv, D] -> out [num_tokens, Hq, D].

        With rope = (inv_freq, interleave), q and k are first rotated at their
        positions (q in place) by the fused prologue kernel; without it they
        are taken as already rotated."""
        if q.shape[0] != self.num_tokens or k.shape[0] != self.num_tokens:
            raise ValueError(f"expected {self.num_tokens} tokens, got q {q.shape[0]}, k {k.shape[0]}")
        if rope is not None:
            inv_freq, interleave = rope
            rope_append_kv(self.pool, layer, self.table, self.q_indptr, q, k, v, inv_freq,
                           interleave)
        else:
            append_kv(self.pool, layer, self.table, self.q_indptr, k, v)
        if out is None:
            out = torch.empty_like(q)
        if self.decode is not None:
            d = self.decode
            if d.tokens is None:
                paged_decode(self.pool, layer, d.table, q, d.plan, self.scale, out=out,
                             workspace=self.workspace)
            else:
                out[d.tokens] = paged_decode(self.pool, layer, d.table,
                                             q.index_select(0, d.tokens).contiguous(), d.plan,
                                             self.scale, workspace=self.workspace)
        if self.prefill is not None:
            p = self.prefill
            if p.tokens is None:
                paged_prefill(self.pool, layer, p.table, p.q_indptr, q, p.plan, self.scale,
                              out=out, workspace=self.workspace)
            else:
                out[p.tokens] = paged_prefill(self.pool, layer, p.table, p.q_indptr,
                                              q.index_select(0, p.tokens).contiguous(), p.plan,
                                              self.scale, workspace=self.workspace)
        return out
