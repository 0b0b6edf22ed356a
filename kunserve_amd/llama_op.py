"""LlamaOp: the KV-cache side of torch.classes.gpt_ops.LlamaOp.

The reference constructs LlamaOp with twelve ints (kunserve/models.py:52-65)
and calls, on the paged-KV path:
  * pforward(...)            kunserve/worker.py:298-312  (attention stage here)
  * local_copy_blocks(...)   kunserve/worker.py:818-823
  * kv_exchange(...)         kunserve/worker.py:514-532  (pack / scatter here)

This class keeps those names, argument orders and meanings. It owns the KV
pool, sized from max_num_pages at construction, exactly as the reference's
LlamaOp owns kv_data (kunserve/models.py:53). The dense parts of pforward
(QKV / O / MLP GEMMs, RoPE, sampling) are outside this library: pforward
here takes the step's host arguments and returns an AttentionStep whose
run(layer, q, k, v) is the per-layer attention stage.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence

import numpy as np
import torch

from .paged_kv import AttentionStep, KVPool, copy_blocks, kv_pack, kv_scatter
from .pmm import PmmPool


def kept_layers(layers: int, rank_in_group: int, num_group_instances: int) -> range:
    """Layers instance rank_in_group of a balloon group of num_group_instances
    keeps: the group splits the model into equal contiguous pipeline stages
    (kunserve/flash_backend.py:2395,2442-2443)."""
    if num_group_instances < 1 or not 0 <= rank_in_group < num_group_instances:
        raise ValueError(f"rank {rank_in_group} outside a group of {num_group_instances}")
    if layers % num_group_instances:
        raise ValueError(f"{layers} layers do not split into {num_group_instances} equal stages")
    per = layers // num_group_instances
    return range(rank_in_group * per, (rank_in_group + 1) * per)


class LlamaOp:
    def __init__(self, max_num_pages: int, layers: int, qo_head: int, kv_head: int,
                 page_size: int, head_size: int, inter_size: int, vocab_size: int,
                 max_batch_size: int, max_batch_tokens: int, max_position_embeddings: int,
                 tensor_parallel_size: int, device: Optional[torch.device] = None,
                 dtype: torch.dtype = torch.float16, max_extend_pages: int = 0):
        if qo_head % kv_head:
            raise ValueError(f"qo_head {qo_head} is not a multiple of kv_head {kv_head}")
        self.max_num_pages = max_num_pages
        self.layers = layers
        self.qo_head = qo_head
        self.kv_head = kv_head
        self.page_size = page_size
        self.head_size = head_size
        self.inter_size = inter_size
        self.vocab_size = vocab_size
        self.max_batch_size = max_batch_size
        self.max_batch_tokens = max_batch_tokens
        self.max_position_embeddings = max_position_embeddings
        self.tensor_parallel_size = tensor_parallel_size
        dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
        # The model dtype (the reference's --dtype, bf16 by default,
        # kunserve/kunserve_config.py:61) is the KV pool's dtype.
        # With max_extend_pages > 0 the pool can grow by the memory of
        # dropped weight layers (pmm_drop); layer_weights() hands out that
        # memory.
        self.num_base_pages = max_num_pages
        self.pmm: Optional[PmmPool] = None
        self._weight_segments: Dict[int, int] = {}   # layer -> segment id
        if max_extend_pages > 0:
            self.pmm = PmmPool(max_num_pages, layers, kv_head, page_size, head_size,
                               max_extend_pages, dev, dtype)
            self.pool = self.pmm.pool
        else:
            self.pool = KVPool.allocate(max_num_pages, layers, kv_head, page_size, head_size,
                                        dev, dtype)

    # -------------------------------------------------------------- pforward

    def pforward(self, num_requests: int, num_tokens: int, max_num_pages: int,
                 local_layer_start: int, local_layer_end: int,
                 input_tokens_batched: List[List[int]], first_token_indexes: List[int],
                 is_prefill_requests: List[int], pages_of_reqs: List[List[int]],
                 num_restore_requests: int = 0, pages_of_pp: Optional[List[List[int]]] = None,
                 pages_of_dp: Optional[List[List[int]]] = None, receiver_rank: int = 0
                 ) -> AttentionStep:
        """Prepares the attention stage of one step (kunserve/worker.py:270-312).

        Argument meanings follow kunserve/flash_backend.py:2448-2469. The
        live-restore arguments (num_restore_requests, pages_of_pp,
        pages_of_dp, receiver_rank) are accepted for signature parity; the
        reference caller passes num_restore_requests = 0
        (kunserve/flash_backend.py:2465).
        """
        if len(input_tokens_batched) != num_requests or len(pages_of_reqs) != num_requests:
            raise ValueError("num_requests does not match the per-row argument lists")
        q_lens = [len(t) for t in input_tokens_batched]
        if sum(q_lens) != num_tokens:
            raise ValueError(f"num_tokens {num_tokens} != {sum(q_lens)} input tokens")
        if not 0 <= local_layer_start <= local_layer_end <= self.layers:
            raise ValueError("local layer range outside the model")
        if max_num_pages > self.max_num_pages:
            raise ValueError(f"max_num_pages {max_num_pages} exceeds the pool "
                             f"({self.max_num_pages})")
        if num_restore_requests:
            raise NotImplementedError("live KV restore inside pforward is not part of this path")
        step = AttentionStep(self.pool, self.qo_head, q_lens, first_token_indexes,
                             is_prefill_requests, pages_of_reqs)
        step.layer_range = (local_layer_start, local_layer_end)
        return step

    # ------------------------------------------------- parameter memory

    def layer_weights(self, layer: int, nbytes: int) -> torch.Tensor:
        """Device memory (uint8, at least nbytes, rounded up to whole block
        pairs) for the weights of one layer, which pmm_drop can turn into KV
        blocks. Valid while the layer is not dropped."""
        if self.pmm is None:
            raise RuntimeError("LlamaOp was built without max_extend_pages")
        if not 0 <= layer < self.layers:
            raise ValueError(f"layer {layer} outside the model")
        if layer not in self._weight_segments:
            self._weight_segments[layer] = self.pmm.add_segment(nbytes)
        elif self.pmm.segment_pages(self._weight_segments[layer]) * 2 * self.pmm.page_bytes < nbytes:
            raise ValueError(f"layer {layer} already holds a smaller weight segment")
        return self.pmm.segment(self._weight_segments[layer])

    def pmm_drop(self, rank_in_group: int, num_group_instances: int) -> int:
        """Drops the weights of every layer outside this instance's stage and
        returns the number of KV blocks they became (kunserve/worker.py:454-458).
        The new blocks are [num_base, num_base + returned) in order of the
        dropped layers (kunserve/block_manager.py:262-269); K blocks take the
        first half of each layer's memory and V blocks the second. Waits for
        the device. Views of the dropped weights must not be used afterwards."""
        if self.pmm is None:
            raise RuntimeError("LlamaOp was built without max_extend_pages")
        keep = kept_layers(self.layers, rank_in_group, num_group_instances)
        dropped = set(self.dropped_layers())
        added = 0
        for layer in sorted(self._weight_segments):
            if layer in keep or layer in dropped:
                continue
            added += len(self.pmm.drop(self._weight_segments[layer]))
        self._sync_pool()
        return added

    def pmm_restore(self) -> List[int]:
        """Maps every dropped layer's memory back to its weights and returns
        those layers (kunserve/worker.py:484-487); their blocks leave the
        pool, so no request may hold them. The memory comes back holding KV
        data: the weights themselves are reloaded by the caller (the
        reference pulls them from a peer instance over NCCL,
        kunserve/llm_engine.py:553-558)."""
        if self.pmm is None:
            raise RuntimeError("LlamaOp was built without max_extend_pages")
        by_segment = {sid: layer for layer, sid in self._weight_segments.items()}
        restored = []
        while self.pmm.dropped:
            restored.append(by_segment[self.pmm.restore()])
        self._sync_pool()
        return sorted(restored)

    def dropped_layers(self) -> List[int]:
        if self.pmm is None:
            return []
        by_segment = {sid: layer for layer, sid in self._weight_segments.items()}
        return sorted(by_segment[s] for s in self.pmm.dropped)

    def _sync_pool(self) -> None:
        self.pool = self.pmm.pool
        self.max_num_pages = self.pmm.num_pages

    # ------------------------------------------------------ block movement

    def local_copy_blocks(self, max_num_pages: int, all_ex_blocks: Sequence[int],
                          all_base_blocks: Sequence[int]) -> None:
        """Copies extend-region blocks into base-region blocks, all layers
        (kunserve/worker.py:818-823; caller kunserve/flash_backend.py:1116-1123)."""
        if len(all_ex_blocks) != len(all_base_blocks):
            raise ValueError("ex and base block lists differ in length")
        ids = np.asarray(list(all_ex_blocks) + list(all_base_blocks), dtype=np.int64)
        if ids.size and (ids.min() < 0 or ids.max() >= min(max_num_pages, self.max_num_pages)):
            raise IndexError(f"block id outside [0, {min(max_num_pages, self.max_num_pages)})")
        if len(set(all_ex_blocks) & set(all_base_blocks)):
            raise ValueError("source and destination blocks overlap")
        copy_blocks(self.pool, all_ex_blocks, all_base_blocks)

    def kv_exchange_pack(self, page_ids: Sequence[int], layer_begin: int, layer_end: int,
                         scratch: Optional[torch.Tensor] = None) -> torch.Tensor:
        """kv_exchange phase 1: gathers the sender's pages (sorted pre-fusion
        local ids, kunserve/flash_backend.py:913-928) for layers
        [layer_begin, layer_end) into one contiguous buffer."""
        return kv_pack(self.pool, layer_begin, layer_end, page_ids, scratch)

    def kv_exchange_scatter(self, page_ids: Sequence[int], layer_begin: int, layer_end: int,
                            scratch: torch.Tensor) -> None:
        """kv_exchange phase 3: writes received pages into fused page ids
        (kunserve/block_manager.py:755-763)."""
        kv_scatter(self.pool, layer_begin, layer_end, page_ids, scratch)

    def kv_exchange(self, pages_of_instances: List[List[int]], pp_rank: int, pp_size: int,
                    group_rank: int, group_size: int, num_base_blocks: int,
                    num_extend_blocks: int) -> None:
        """kunserve/worker.py:514-532. With group_size == 1 nothing moves.
        A multi-instance exchange needs the RCCL transport between the pack
        and scatter phases, which runs on more than one GPU and is not part
        of this single-GPU library."""
        if group_size <= 1:
            return
        raise NotImplementedError(
            "kv_exchange across instances needs RCCL send/recv between kv_exchange_pack and "
            "kv_exchange_scatter; only the single-GPU pack/scatter phases are provided")
