"""ctypes binding of libkunserve_hip.so (declared in include/kunserve_hip.h).

The library is loaded once, from the package directory. There is no fallback:
if the library is missing, every entry point raises.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, Structure, c_float, c_int, c_int32, c_int64, c_void_p, c_char_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libkunserve_hip.so"

# Error codes of include/kunserve_hip.h.
OK = 0
EINVAL = -1
ERANGE = -2
ENOSPC = -3
EUNSUPPORTED = -4
EHIP = -5
_CODE_NAMES = {EINVAL: "EINVAL", ERANGE: "ERANGE", ENOSPC: "ENOSPC",
               EUNSUPPORTED: "EUNSUPPORTED", EHIP: "EHIP"}


class KVPool(Structure):
    _fields_ = [
        ("k", c_void_p), ("v", c_void_p),
        ("num_pages", c_int64), ("page_stride", c_int64), ("layer_stride", c_int64),
        ("head_stride", c_int64), ("token_stride", c_int64),
        ("num_layers", c_int32), ("num_kv_heads", c_int32),
        ("page_size", c_int32), ("head_dim", c_int32), ("dtype", c_int32),
    ]


DTYPE_F16 = 0    # KUNSERVE_DTYPE_F16
DTYPE_BF16 = 1   # KUNSERVE_DTYPE_BF16


class PageTable(Structure):
    _fields_ = [
        ("indptr_dev", c_void_p), ("indices_dev", c_void_p), ("kv_len_dev", c_void_p),
        ("num_seqs", c_int32),
    ]


class Tensor3(Structure):
    _fields_ = [("data", c_void_p), ("token_stride", c_int64), ("head_stride", c_int64)]


class DecodePlanInfo(Structure):
    _fields_ = [
        ("num_work", c_int32), ("num_merge", c_int32), ("num_slots", c_int32),
        ("part_tokens", c_int32), ("group_size", c_int32), ("plan_ints", c_int32),
    ]


class PrefillPlanInfo(Structure):
    _fields_ = [("num_tiles", c_int32), ("tile_q", c_int32), ("plan_ints", c_int32),
                ("num_qo_heads", c_int32), ("max_kv_len", c_int32), ("num_merge", c_int32),
                ("num_slots", c_int32), ("kv_chunk", c_int32), ("head_dim", c_int32)]


# name -> (restype, argtypes); must match include/kunserve_hip.h.
SIGNATURES = {
    "kunserve_version": (c_int32, []),
    "kunserve_last_error": (c_char_p, []),
    "kunserve_copy_blocks": (c_int, [POINTER(KVPool), c_void_p, c_void_p, c_int64, c_void_p]),
    "kunserve_kv_pack": (c_int, [POINTER(KVPool), c_int32, c_int32, c_void_p, c_int64,
                                 c_void_p, c_int64, c_void_p]),
    "kunserve_kv_scatter": (c_int, [POINTER(KVPool), c_int32, c_int32, c_void_p, c_int64,
                                    c_void_p, c_int64, c_void_p]),
    "kunserve_kv_pack_bytes": (c_int64, [POINTER(KVPool), c_int32, c_int64]),
    "kunserve_hbm_probe": (c_int, [c_int32, c_void_p, c_void_p, c_int64, c_void_p]),
    "kunserve_decode_slab_probe": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32,
                                           c_int64, c_int32, c_int32, c_void_p, c_void_p]),
    "kunserve_mfma_probe": (c_int, [c_int32, c_void_p, c_void_p, c_int32, c_int32, c_void_p]),
    "kunserve_swap_blocks": (c_int, [c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_void_p,
                                     c_int64, c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "kunserve_append_kv": (c_int, [POINTER(KVPool), c_int32, POINTER(PageTable), c_void_p,
                                   c_int32, POINTER(Tensor3), POINTER(Tensor3), c_void_p]),
    "kunserve_rope_append_kv": (c_int, [POINTER(KVPool), c_int32, POINTER(PageTable), c_void_p,
                                        c_int32, POINTER(Tensor3), c_int32, POINTER(Tensor3),
                                        POINTER(Tensor3), c_void_p, c_int32, c_void_p]),
    "kunserve_decode_plan_bound": (c_int64, [c_void_p, c_int32]),
    "kunserve_decode_plan": (c_int, [c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32,
                                     c_void_p, c_int64, POINTER(DecodePlanInfo)]),
    "kunserve_decode_workspace_bytes": (c_int64, [POINTER(DecodePlanInfo), c_int32, c_int32]),
    "kunserve_paged_decode": (c_int, [POINTER(KVPool), c_int32, POINTER(PageTable), c_void_p,
                                      POINTER(Tensor3), POINTER(Tensor3), c_int32, c_float,
                                      c_void_p, POINTER(DecodePlanInfo), c_void_p, c_int64,
                                      c_void_p]),
    "kunserve_paged_decode_noalloc_max_bytes": (c_int64, []),
    "kunserve_paged_decode_noalloc": (c_int, [POINTER(KVPool), c_int32, POINTER(PageTable),
                                              c_void_p, POINTER(Tensor3), POINTER(Tensor3),
                                              c_int32,
                                              c_float, c_void_p, POINTER(DecodePlanInfo),
                                              c_void_p]),
    "kunserve_prefill_plan_bound": (c_int64, [c_void_p, c_int32, c_int32, c_int32]),
    "kunserve_prefill_plan": (c_int, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32,
                                      c_int32, c_void_p, c_int64, POINTER(PrefillPlanInfo)]),
    "kunserve_prefill_workspace_bytes": (c_int64, [POINTER(PrefillPlanInfo)]),
    "kunserve_paged_prefill": (c_int, [POINTER(KVPool), c_int32, POINTER(PageTable), c_void_p,
                                       c_void_p, POINTER(Tensor3), POINTER(Tensor3), c_int32, c_float,
                                       c_void_p, POINTER(PrefillPlanInfo), c_void_p, c_int64,
                                       c_void_p]),
    "kunserve_fused_pool": (c_int, [POINTER(KVPool), c_int64, c_int32, POINTER(KVPool)]),
    "kunserve_fused_page_ids": (c_int, [c_void_p, c_int64, c_int64, c_int32, c_int64,
                                        c_void_p]),
    "kunserve_pmm_create": (c_int, [c_int32, c_int64, c_int64, c_int64, POINTER(c_void_p)]),
    "kunserve_pmm_add_segment": (c_int, [c_void_p, c_int64, POINTER(c_int32),
                                         POINTER(c_void_p)]),
    "kunserve_pmm_drop": (c_int, [c_void_p, c_int32, POINTER(c_int64)]),
    "kunserve_pmm_restore": (c_int, [c_void_p, POINTER(c_int32), POINTER(c_int64)]),
    "kunserve_pmm_pools": (c_int, [c_void_p, POINTER(c_void_p), POINTER(c_void_p),
                                   POINTER(c_int64)]),
    "kunserve_pmm_destroy": (None, [c_void_p]),
}

_lib: ctypes.CDLL | None = None


class KunserveError(RuntimeError):
    """A C ABI call returned a non-zero status."""

    def __init__(self, func: str, code: int, message: str):
        super().__init__(f"{func} failed ({_CODE_NAMES.get(code, code)}): {message}")
        self.code = code


def lib() -> ctypes.CDLL:
    """Loads the HIP library (once) and declares its signatures."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m kunserve_amd.build`"
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def call(name: str, *args) -> int:
    """Calls `name`; raises KunserveError on a negative status."""
    fn = getattr(lib(), name)
    rc = fn(*args)
    if rc < 0:
        msg = lib().kunserve_last_error()
        raise KunserveError(name, rc, msg.decode() if msg else "")
    return rc
