"""MI355X (gfx950) paged-KV attention path for KunServe.

Importing the package registers torch.ops.swapping_ops.swap with the
reference schema (kunserve/worker.py:673-681), backed by the HIP library, so
the reference's ParaWorker.swap_blocks call runs unchanged. LlamaOp mirrors
the KV-cache side of torch.classes.gpt_ops.LlamaOp (kunserve/models.py:52-65),
and importing the package also makes that name resolve to it, so the
reference's constructor call (12 ints) runs unchanged.
"""
from __future__ import annotations

import types

import torch

from . import _lib
from .llama_op import LlamaOp, kept_layers
from .paged_kv import (AttentionStep, DecodePlan, KVPool, PageTable, PrefillPlan, append_kv,
                       copy_blocks, csr_from_lists, kv_lens_for_step, kv_pack, kv_scatter,
                       paged_decode, paged_prefill, rope_append_kv, rope_inv_freq, swap)
from .pmm import PmmPool

__all__ = [
    "AttentionStep", "DecodePlan", "KVPool", "LlamaOp", "PageTable", "PmmPool", "PrefillPlan",
    "append_kv", "copy_blocks", "csr_from_lists", "kv_lens_for_step", "kv_pack",
    "kept_layers", "kv_scatter", "paged_decode", "paged_prefill", "rope_append_kv", "rope_inv_freq", "swap",
    "library_path",
]


def library_path() -> str:
    return str(_lib.LIB_PATH)


def _register_swapping_ops() -> None:
    if hasattr(torch.ops, "swapping_ops") and hasattr(torch.ops.swapping_ops, "swap"):
        return
    lib = torch.library.Library("swapping_ops", "DEF")
    lib.define("swap(int[] source_block_ids, int[] target_block_ids, bool is_swap_in, "
               "Tensor k_cache, Tensor v_cache, Tensor k_swap, Tensor v_swap) -> ()")

    def _swap_impl(source_block_ids, target_block_ids, is_swap_in, k_cache, v_cache, k_swap,
                   v_swap):
        swap(source_block_ids, target_block_ids, is_swap_in, k_cache, v_cache, k_swap, v_swap)

    lib.impl("swap", _swap_impl, "CompositeExplicitAutograd")
    globals()["_swapping_ops_lib"] = lib


try:
    _register_swapping_ops()
except RuntimeError:
    # Already defined by another loader in this process.
    pass


class _GptOpsNamespace(types.ModuleType):
    """torch.classes.gpt_ops with LlamaOp bound to this package's class;
    every other name is looked up among the natively registered classes."""

    def __init__(self, native):
        super().__init__("torch.classes.gpt_ops")
        self._native = native
        self.LlamaOp = LlamaOp

    def __getattr__(self, name):
        return getattr(self._native, name)


def _register_gpt_ops() -> None:
    """torch.classes resolves `torch.classes.<ns>.<Class>` through the C++
    custom-class registry and caches the namespace object on torch.classes.
    When no native gpt_ops.LlamaOp is registered, the cached namespace is
    replaced by one whose LlamaOp is this package's class (a native one, if
    a library registered it, is left in place)."""
    native = torch.classes.gpt_ops
    try:
        native.LlamaOp
        return
    except RuntimeError:
        pass
    setattr(torch.classes, "gpt_ops", _GptOpsNamespace(native))


_register_gpt_ops()
