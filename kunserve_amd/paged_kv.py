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
from typing import Callable, Optional, Sequence

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


def _upload(arr: np.ndarray, device: torch.device) -> torch.Tensor:
    """A new device tensor holding `arr`, enqueued on the current stream with
    no host wait: the bytes go through a pinned buffer of torch's caching
    host allocator, which keeps that buffer from reuse until the copy ran."""
    src = torch.from_numpy(np.ascontiguousarray(arr))
    staged = torch.empty(src.shape, dtype=src.dtype, pin_memory=True)
    staged.copy_(src)
    return staged.to(device, non_blocking=True)


def _upload_packed(arrays: Sequence[np.ndarray], device: torch.device) -> list:
    """Uploads several int32 host arrays with one copy; returns a device
    view per array (all views share one allocation)."""
    sizes = [int(a.size) for a in arrays]
    dev = _upload(np.concatenate([_i32(a).reshape(-1) for a in arrays]) if arrays
                  else np.zeros(0, np.int32), device)
    out, at = [], 0
    for n in sizes:
        out.append(dev[at:at + n])
        at += n
    return out


_DTYPES = {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16}


_V_OFFSET_ELEMS = 2048   # 4 KiB of 16-bit elements


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
        # V starts 4 KiB into its allocation. Decode loads the K and the V slab
        # of a (page, layer, head) back to back; offset this way they are
        # served about 1% faster (Llama-2-7B decode: 142.6-142.7 against
        # 143.9 us per launch with V at its allocation's start; 1 KiB measured
        # the same, 256 bytes and 2 KiB in between).
        n = math.prod(shape)
        v = torch.empty(n + _V_OFFSET_ELEMS, dtype=dtype, device=device)
        return cls(torch.empty(shape, dtype=dtype, device=device),
                   v[_V_OFFSET_ELEMS:].view(shape))

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

    def fused_view(self, base_pages: int, fusion_size: int) -> "KVPool":
        """The pool as a fusion group of `fusion_size` instances addresses it
        (kunserve/block_manager.py:231-269): each page of L layers becomes
        fusion_size pages of L / fusion_size layers. Layer group i of base
        page b is fused page i * base_pages + b, and page base_pages + q of
        the extend region (pages past the base ones) holds fused extend pages
        base_pages * fusion_size + q * fusion_size + i. Nothing is copied: the
        view has num_pages * fusion_size pages of L / fusion_size layers over
        the same memory (kunserve_fused_pool), and fused ids are turned into
        its page indices by fused_page_ids."""
        desc = _lib.KVPool()
        _lib.call("kunserve_fused_pool", ctypes.byref(self._desc), base_pages, fusion_size,
                  ctypes.byref(desc))
        shape = (desc.num_pages, desc.num_layers, self.num_kv_heads, self.page_size,
                 self.head_dim)
        strides = (desc.page_stride, desc.layer_stride) + tuple(self.k.stride()[2:])
        k = self.k.as_strided(shape, strides, self.k.storage_offset())
        v = self.v.as_strided(shape, strides, self.v.storage_offset())
        view = KVPool(k, v, owner=self._owner)
        view._generation = self._generation
        view.base_pages, view.fusion_size = base_pages, fusion_size
        return view


def fused_page_ids(ids, base_pages: int, fusion_size: int, num_fused_pages: int) -> np.ndarray:
    """Fused page ids (kunserve/block_manager.py:250-253,262-269) -> pages of
    KVPool.fused_view(base_pages, fusion_size) (kunserve_fused_page_ids)."""
    arr = _i32(ids).reshape(-1)
    out = np.empty_like(arr)
    _lib.call("kunserve_fused_page_ids", arr.ctypes.data, arr.size, base_pages, fusion_size,
              num_fused_pages, out.ctypes.data)
    return out


# ------------------------------------------------------------ step arguments


def kv_lens_for_step(first_token_indexes: Sequence[int], q_lens: Sequence[int],
                     is_prefill_requests: Sequence[int], use_tensor_cores: bool = False,
                     is_context_stage: Optional[Sequence[int]] = None,
                     pages_per_row: Optional[Sequence[int]] = None,
                     page_size: int = 0) -> np.ndarray:
    """KV length of each row after this step's tokens are appended.

    kunserve/request.py:447-462: a prefill row's first index is
    prefill_begin_index (tokens already cached), so kv_len = first + q_len;
    a decode row's first index is prompt_len + output_len, which already
    counts the token being decoded (the block allocation of
    kunserve/request.py:414-423 and kunserve/block_manager.py:493-500 uses
    the same count), so kv_len = first. In both cases the new tokens occupy
    positions [kv_len - q_len, kv_len).

    With use_tensor_cores every row arrives flagged as prefill
    (kunserve/request.py:667-670, kunserve/flash_backend.py:2460-2462), so
    the flag no longer tells a decode row from a one-token prefill chunk.
    The caller then passes the rows' real stages as is_context_stage
    ([int(r.is_context_stage()) for r in requests]), which decide every
    row. Without them, rows of several tokens are prefill rows and a
    one-token row at first index 0 is the chunk of a one-token prompt; a
    one-token row at first index f > 0 is a decode row only if its page
    list (pages_per_row, of page_size tokens) is too short to hold position
    f, which the table of a prefill chunk, cut to ceil((f + 1) / page_size)
    pages (kunserve/block_manager.py:786-795), always holds. Any other such
    row could be either (the last chunk of a prompt one token longer than a
    chunk multiple, or a decode row), and guessing would write its K/V one
    position off: ValueError.
    """
    first = np.asarray(first_token_indexes, dtype=np.int64)
    ql = np.asarray(q_lens, dtype=np.int64)
    decode = decode_rows(first_token_indexes, q_lens, is_prefill_requests, use_tensor_cores,
                         is_context_stage, pages_per_row, page_size)
    if np.any(decode & (ql != 1)):
        bad = int(np.argmax(decode & (ql != 1)))
        raise ValueError(f"row {bad}: a decode row takes exactly one input token, got {ql[bad]}")
    kv = np.where(decode, first, first + ql)
    if np.any(kv < ql):
        bad = int(np.argmax(kv < ql))
        raise ValueError(f"row {bad}: kv_len {kv[bad]} shorter than its {ql[bad]} new tokens")
    return kv.astype(np.int32)


def decode_rows(first_token_indexes: Sequence[int], q_lens: Sequence[int],
                is_prefill_requests: Sequence[int], use_tensor_cores: bool = False,
                is_context_stage: Optional[Sequence[int]] = None,
                pages_per_row: Optional[Sequence[int]] = None,
                page_size: int = 0) -> np.ndarray:
    """Boolean mask of the decode rows of a step, by the rule of
    kv_lens_for_step (which raises where this does)."""
    first = np.asarray(first_token_indexes, dtype=np.int64)
    ql = np.asarray(q_lens, dtype=np.int64)
    flag = np.asarray(is_prefill_requests, dtype=np.int64)
    if not (first.shape == ql.shape == flag.shape):
        raise ValueError("first_token_indexes, q_lens and is_prefill_requests differ in length")
    if is_context_stage is not None:
        stage = np.asarray(is_context_stage, dtype=np.int64)
        if stage.shape != first.shape:
            raise ValueError("is_context_stage differs in length from the other row arguments")
        return stage == 0
    if not use_tensor_cores:
        return flag == 0
    open_rows = (flag != 0) & (ql == 1) & (first > 0)
    settled = np.zeros_like(open_rows)
    if pages_per_row is not None:
        pages = np.asarray(pages_per_row, dtype=np.int64)
        if pages.shape != first.shape:
            raise ValueError("pages_per_row differs in length from the other row arguments")
        if page_size <= 0:
            raise ValueError("pages_per_row needs the page_size")
        settled = open_rows & (pages * page_size <= first)
    if np.any(open_rows & ~settled):
        bad = int(np.argmax(open_rows & ~settled))
        raise ValueError(
            f"row {bad}: with use_tensor_cores every row is flagged as prefill, and a one-token "
            f"row at first index {int(first[bad])} may be a decode row or the last chunk of a "
            f"prompt; pass is_context_stage (each row's request.is_context_stage())")
    return (flag == 0) | settled


def csr_from_lists(pages_of_reqs: Sequence[Sequence[int]], kv_len: np.ndarray,
                   page_size: int, num_pages: int,
                   id_map: Optional[Callable[[np.ndarray], np.ndarray]] = None
                   ) -> tuple[np.ndarray, np.ndarray]:
    """Ragged page lists -> (indptr, indices) int32, validated.

    Each row must hold at least ceil(kv_len / page_size) pages
    (kunserve/block_manager.py:493-500,786-795); only those are kept. Ids
    must lie in [0, num_pages); id_map, if given, then turns them into the
    page indices the kernels use (fused ids -> pages of a fused view).
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
    indices = indices.astype(np.int32)
    if id_map is not None:
        indices = _i32(id_map(indices))
    return indptr.astype(np.int32), indices


class PageTable:
    """Per-step CSR page table, on the device and mirrored on the host.

    The device copy is enqueued on the current stream through pinned memory
    (no host wait). With upload=False nothing is copied until bind() is given
    device views of host_arrays() (AttentionStep uploads all of a step's
    arrays with one copy)."""

    def __init__(self, indptr: np.ndarray, indices: np.ndarray, kv_len: np.ndarray,
                 device: torch.device, upload: bool = True):
        self.indptr_host = _i32(indptr)
        self.indices_host = _i32(indices)
        self.kv_len_host = _i32(kv_len)
        self.num_seqs = len(self.kv_len_host)
        self.device = device
        if len(self.indptr_host) != self.num_seqs + 1:
            raise ValueError("indptr must have num_seqs + 1 entries")
        self._desc = None
        if upload:
            self.bind(_upload_packed(self.host_arrays(), device))

    def host_arrays(self) -> list:
        return [self.indptr_host, self.kv_len_host, self.indices_host]

    def bind(self, dev: Sequence[torch.Tensor]) -> None:
        self.indptr, self.kv_len, self.indices = dev
        self._desc = _lib.PageTable(self.indptr.data_ptr(), self.indices.data_ptr(),
                                    self.kv_len.data_ptr(), self.num_seqs)

    @classmethod
    def from_lists(cls, pages_of_reqs: Sequence[Sequence[int]], kv_len, pool: KVPool,
                   id_map: Optional[Callable[[np.ndarray], np.ndarray]] = None,
                   num_ids: Optional[int] = None, upload: bool = True) -> "PageTable":
        """num_ids: bound of the ids the lists may hold (default: the pool's
        pages); id_map turns valid ids into pool pages."""
        kv = _i32(kv_len)
        indptr, indices = csr_from_lists(pages_of_reqs, kv, pool.page_size,
                                         pool.num_pages if num_ids is None else num_ids, id_map)
        return cls(indptr, indices, kv, pool.device, upload)

    def desc(self):
        if self._desc is None:
            raise RuntimeError("page table used before its device arrays were bound")
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
                 device: torch.device, part_tokens: int = 0, num_cus: Optional[int] = None,
                 upload: bool = True):
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
        self.plan = None
        if upload:
            self.bind(_upload_packed(self.host_arrays(), device))
        self.num_qo_heads = num_qo_heads
        self.num_kv_heads = num_kv_heads

    def host_arrays(self) -> list:
        return [self.plan_host]

    @property
    def num_items(self) -> int:
        """Work items (partitions) of the plan, without the lanes' padding."""
        return int((self.plan_host[: 4 * self.info.num_work: 4] >= 0).sum())

    def bind(self, dev: Sequence[torch.Tensor]) -> None:
        self.plan = dev[0] if self.info.plan_ints else None

    def workspace_bytes(self, head_dim: int) -> int:
        return int(_lib.lib().kunserve_decode_workspace_bytes(
            ctypes.byref(self.info), self.num_qo_heads, head_dim))


class PrefillPlan:
    """(row, q tile, q head) work items of the prefill rows, XCD-ordered
    (kunserve_prefill_plan). Steps with too few items to fill the device
    split each item's KV range; the merge runs inside paged_prefill."""

    def __init__(self, q_indptr_host: Sequence[int], kv_len_host: Sequence[int],
                 num_qo_heads: int, num_kv_heads: int, device: torch.device,
                 num_cus: Optional[int] = None, upload: bool = True, head_dim: int = 128):
        """head_dim: the pool's (64, 128 or 256); it sets the plan's tile."""
        qi = _i32(q_indptr_host)
        kv = _i32(kv_len_host)
        n = len(kv)
        if len(qi) != n + 1:
            raise ValueError("q_indptr must have num_seqs + 1 entries")
        cap = int(_lib.lib().kunserve_prefill_plan_bound(qi.ctypes.data, n, num_qo_heads,
                                                         head_dim))
        # A negative bound (bad arguments) leaves the plan call to report them.
        buf = np.zeros(max(cap, 3), dtype=np.int32)
        self.info = _lib.PrefillPlanInfo()
        cus = num_cus if num_cus is not None else _num_cus(device)
        _lib.call("kunserve_prefill_plan", qi.ctypes.data, kv.ctypes.data if n else None, n,
                  num_qo_heads, num_kv_heads, head_dim, cus, buf.ctypes.data, buf.size,
                  ctypes.byref(self.info))
        self.plan_host = buf[: self.info.plan_ints].copy()
        self.plan = None
        if upload:
            self.bind(_upload_packed(self.host_arrays(), device))

    def host_arrays(self) -> list:
        return [self.plan_host]

    def bind(self, dev: Sequence[torch.Tensor]) -> None:
        self.plan = dev[0] if self.info.plan_ints else None

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
    return _upload(arr.astype(np.int32), pool.device)


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
    return _upload(t.numpy(), device) if device is not None else t


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


def _check_row_map(m: Optional[torch.Tensor], n: int, device: torch.device, what: str) -> None:
    if m is not None and (m.dtype != torch.int32 or m.shape != (n,) or m.device != device
                          or not m.is_contiguous()):
        raise ValueError(f"{what} must be a contiguous int32 tensor of {n} entries on {device}")


def paged_decode(pool: KVPool, layer: int, table: PageTable, q: torch.Tensor, plan: DecodePlan,
                 sm_scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
                 workspace: Optional[torch.Tensor] = None,
                 q_token: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Decode attention of q [num_seqs, Hq, D] over each row's pages.

    With q_token (device int32 [num_seqs], each entry < q.shape[0]), row b's
    query and output are token q_token[b] of q and out ([num_tokens, Hq, D]):
    the decode rows of a mixed step, read and written in place."""
    hq = q.shape[1]
    if q_token is None and q.shape[0] != table.num_seqs:
        raise ValueError(f"q has {q.shape[0]} tokens for {table.num_seqs} rows")
    if q.shape[2] != pool.head_dim:
        raise ValueError(f"q shape {tuple(q.shape)} does not match head_dim {pool.head_dim}")
    _check_row_map(q_token, table.num_seqs, q.device, "q_token")
    if out is None:
        out = torch.empty_like(q)
    if out.shape != q.shape:
        raise ValueError(f"out shape {tuple(out.shape)} differs from q's {tuple(q.shape)}")
    pool.check_dtype(q, out)
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(pool.head_dim)
    need = plan.workspace_bytes(pool.head_dim)
    if need > 0 and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=pool.device)
    qd, od = _tensor3(q), _tensor3(out)
    _lib.call("kunserve_paged_decode", pool.desc(), layer, table.desc(), _ptr(q_token),
              ctypes.byref(qd), ctypes.byref(od), hq, ctypes.c_float(scale),
              _ptr(plan.plan), ctypes.byref(plan.info), _ptr(workspace),
              0 if workspace is None else workspace.numel() * workspace.element_size(),
              _stream_ptr(pool.device))
    return out


def paged_prefill(pool: KVPool, layer: int, table: PageTable, q_indptr: torch.Tensor,
                  q: torch.Tensor, plan: PrefillPlan, sm_scale: Optional[float] = None,
                  out: Optional[torch.Tensor] = None,
                  workspace: Optional[torch.Tensor] = None,
                  q_start: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Causal chunked-prefill attention of ragged q [num_tokens, Hq, D].

    Row b has q_indptr[b+1] - q_indptr[b] tokens, at q_indptr[b] onwards, or
    with q_start (device int32 [num_seqs]) at q_start[b] onwards: the
    prefill rows of a mixed step, read and written in place."""
    _check_row_map(q_start, table.num_seqs, q.device, "q_start")
    if out is None:
        out = torch.empty_like(q)
    if out.shape != q.shape:
        raise ValueError(f"out shape {tuple(out.shape)} differs from q's {tuple(q.shape)}")
    pool.check_dtype(q, out)
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(pool.head_dim)
    need = plan.workspace_bytes()
    if need > 0 and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=pool.device)
    qd, od = _tensor3(q), _tensor3(out)
    _lib.call("kunserve_paged_prefill", pool.desc(), layer, table.desc(), q_indptr.data_ptr(),
              _ptr(q_start), ctypes.byref(qd), ctypes.byref(od), q.shape[1], ctypes.c_float(scale),
              _ptr(plan.plan), ctypes.byref(plan.info), _ptr(workspace),
              0 if workspace is None else workspace.numel() * workspace.element_size(),
              _stream_ptr(pool.device))
    return out


@dataclass
class _Subset:
    rows: np.ndarray            # row indices into the batch
    # int32 per subset row: its (first) token in q and out; None when the
    # subset is the whole step, whose rows' tokens are in order
    tokens: Optional[torch.Tensor]
    table: PageTable
    q_indptr: Optional[torch.Tensor]
    plan: object


class AttentionStep:
    """The attention stage of one LlamaOp.pforward step, prepared once from
    the step's host arguments and run for every layer.

    Per layer: append the new K/V of every row, then decode attention for
    decode rows and causal chunked-prefill attention for the others. Which
    rows decode follows kv_lens_for_step (flag 0; with use_tensor_cores,
    where every row is flagged, kunserve/request.py:667-670, the rows' real
    stages, is_context_stage, and a step whose one-token rows they do not
    settle raises ValueError).

    pool may be a fused view (KVPool.fused_view); id_map then turns the
    page lists' fused ids into its pages, and num_ids bounds those ids.
    run(layer, ...) addresses pool layer layer - layer_offset, so a fused
    stage runs its global layer indices on its local layers.

    All of the step's index arrays (tables, plans, row and token indices)
    reach the device in one copy on the current stream, with no host wait.
    """

    def __init__(self, pool: KVPool, num_qo_heads: int, q_lens: Sequence[int],
                 first_token_indexes: Sequence[int], is_prefill_requests: Sequence[int],
                 pages_of_reqs: Sequence[Sequence[int]], sm_scale: Optional[float] = None,
                 decode_part_tokens: int = 0, use_tensor_cores: bool = False,
                 is_context_stage: Optional[Sequence[int]] = None, layer_offset: int = 0,
                 id_map: Optional[Callable[[np.ndarray], np.ndarray]] = None,
                 num_ids: Optional[int] = None):
        self.pool = pool
        self.num_qo_heads = num_qo_heads
        self.layer_offset = layer_offset
        dev = pool.device
        q_lens = np.asarray(q_lens, dtype=np.int64)
        if len(pages_of_reqs) != len(q_lens):
            raise ValueError(f"{len(q_lens)} rows but {len(pages_of_reqs)} page lists")
        if np.any(q_lens < 1):
            raise ValueError("every row needs at least one input token")
        pages_per_row = [len(p) for p in pages_of_reqs]
        self.kv_len = kv_lens_for_step(first_token_indexes, q_lens, is_prefill_requests,
                                       use_tensor_cores, is_context_stage, pages_per_row,
                                       pool.page_size)
        is_decode = decode_rows(first_token_indexes, q_lens, is_prefill_requests,
                                use_tensor_cores, is_context_stage, pages_per_row,
                                pool.page_size)
        self.q_indptr_host = np.zeros(len(q_lens) + 1, dtype=np.int32)
        np.cumsum(q_lens, out=self.q_indptr_host[1:])
        self.num_tokens = int(self.q_indptr_host[-1])
        n_rows = len(q_lens)
        self.table = PageTable.from_lists(pages_of_reqs, self.kv_len, pool, id_map, num_ids,
                                          upload=False)
        self.scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(pool.head_dim)
        if not (math.isfinite(self.scale) and self.scale > 0):
            raise ValueError(f"sm_scale {self.scale} must be finite and positive")

        # Host side of every device array of the step; uploaded together below.
        uploads = [[self.q_indptr_host], self.table]
        self.decode = self.prefill = None
        all_rows = np.arange(n_rows)
        dec_rows, pre_rows = all_rows[is_decode], all_rows[~is_decode]
        # Row subsets take their rows from the step's CSR arrays (ids already
        # checked and mapped), not from the lists again.
        def sub_table(rows):
            lo, hi = self.table.indptr_host[rows], self.table.indptr_host[rows + 1]
            indptr = np.concatenate([[0], np.cumsum(hi - lo)]).astype(np.int32)
            indices = (np.concatenate([self.table.indices_host[a:b] for a, b in zip(lo, hi)])
                       if rows.size else np.zeros(0, np.int32))
            return PageTable(indptr, indices, self.kv_len[rows], dev, upload=False)

        if dec_rows.size:
            whole = dec_rows.size == n_rows
            table = self.table if whole else sub_table(dec_rows)
            tokens = None if whole else self.q_indptr_host[dec_rows].astype(np.int32)
            plan = DecodePlan(self.kv_len[dec_rows], num_qo_heads, pool.num_kv_heads, dev,
                              part_tokens=decode_part_tokens, upload=False)
            self.decode = _Subset(dec_rows, tokens, table, None, plan)
            uploads += ([] if whole else [table, [tokens]]) + [plan]
        if pre_rows.size:
            whole = pre_rows.size == n_rows
            if whole:
                table, tokens, qi = self.table, None, self.q_indptr_host
            else:
                table = sub_table(pre_rows)
                tokens = self.q_indptr_host[pre_rows].astype(np.int32)
                qi = np.zeros(pre_rows.size + 1, dtype=np.int32)
                np.cumsum(q_lens[pre_rows], out=qi[1:])
            plan = PrefillPlan(qi, self.kv_len[pre_rows], num_qo_heads, pool.num_kv_heads, dev,
                               upload=False, head_dim=pool.head_dim)
            self.prefill = _Subset(pre_rows, tokens, table, None, plan)
            uploads += ([] if whole else [table, [tokens], [qi]]) + [plan]

        # One copy for all of them.
        flat, owners = [], []
        for u in uploads:
            arrays = u if isinstance(u, list) else u.host_arrays()
            owners.append((u, len(arrays)))
            flat += arrays
        views = _upload_packed(flat, dev)
        at = 0
        bound = []
        for u, n in owners:
            part = views[at:at + n]
            at += n
            if isinstance(u, list):
                bound.append(part)
            else:
                u.bind(part)
        self.q_indptr = bound[0][0]
        rest = iter(bound[1:])
        if self.decode is not None and self.decode.tokens is not None:
            self.decode.tokens = next(rest)[0]
        if self.prefill is not None:
            if self.prefill.tokens is not None:
                self.prefill.tokens = next(rest)[0]
                self.prefill.q_indptr = next(rest)[0]
            else:
                self.prefill.q_indptr = self.q_indptr
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
        local = layer - self.layer_offset
        if not 0 <= local < self.pool.num_layers:
            raise ValueError(f"layer {layer} outside this step's layers "
                             f"[{self.layer_offset}, {self.layer_offset + self.pool.num_layers})")
        if rope is not None:
            inv_freq, interleave = rope
            rope_append_kv(self.pool, local, self.table, self.q_indptr, q, k, v, inv_freq,
                           interleave)
        else:
            append_kv(self.pool, local, self.table, self.q_indptr, k, v)
        if out is None:
            out = torch.empty_like(q)
        # Each kernel reads its rows' q and writes their out in place: in a
        # mixed step through the subset's row -> token map.
        if self.decode is not None:
            d = self.decode
            paged_decode(self.pool, local, d.table, q, d.plan, self.scale, out=out,
                         workspace=self.workspace, q_token=d.tokens)
        if self.prefill is not None:
            p = self.prefill
            paged_prefill(self.pool, local, p.table, p.q_indptr, q, p.plan, self.scale,
                          out=out, workspace=self.workspace, q_start=p.tokens)
        return out
