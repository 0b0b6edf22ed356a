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

Page ids follow the reference's block manager in both of its states:
  * unfused: ids [0, P) name pages of all layers (P = max_num_pages);
  * fused (a balloon group of N instances, kunserve/block_manager.py:231-269):
    a pforward over one pipeline stage (local layers [r*G, (r+1)*G),
    G = layers / N, kunserve/flash_backend.py:2442-2443) takes fused ids:
    i*P + b is layer group i of base page b, and ids from P*N on are the
    extend pages pmm_drop made, G layers each. The stage's layers live in
    those G-layer pages, so a stale request that keeps id r*P + b
    (kunserve/block_manager.py:755-760) reads the bytes page b held, with no
    copy (KVPool.fused_view).
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence

import numpy as np
import torch

from .paged_kv import (AttentionStep, KVPool, copy_blocks, fused_page_ids, kv_pack,
                       kv_scatter)
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
                 dtype: torch.dtype = torch.float16, max_extend_pages: int = 0,
                 use_tensor_cores: bool = False):
        """use_tensor_cores: the engine's --use-tensor-cores
        (kunserve/kunserve_config.py:54-55), under which every row arrives
        flagged as prefill (see kv_lens_for_step)."""
        if qo_head % kv_head:
            raise ValueError(f"qo_head {qo_head} is not a multiple of kv_head {kv_head}")
        self.use_tensor_cores = use_tensor_cores
        # Instances in the balloon group this op last joined (pmm_drop).
        self.fusion_size = 1
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
                 pages_of_dp: Optional[List[List[int]]] = None, receiver_rank: int = 0,
                 is_context_stage: Optional[List[int]] = None) -> AttentionStep:
        """Prepares the attention stage of one step (kunserve/worker.py:270-312).

        Argument meanings follow kunserve/flash_backend.py:2448-2469. A layer
        range that is one pipeline stage of the model (fusion execution,
        kunserve/flash_backend.py:2442-2443) takes fused page ids below
        max_num_pages = P*N + E (kunserve/flash_backend.py:2435-2440); the
        whole model takes unfused ids. The live-restore arguments
        (num_restore_requests, pages_of_pp, pages_of_dp, receiver_rank) are
        accepted for signature parity; the reference caller passes
        num_restore_requests = 0 (kunserve/flash_backend.py:2465).
        is_context_stage (not in the reference signature) gives the rows'
        real stages when use_tensor_cores hides them (kv_lens_for_step).
        """
        if len(input_tokens_batched) != num_requests or len(pages_of_reqs) != num_requests:
            raise ValueError("num_requests does not match the per-row argument lists")
        q_lens = [len(t) for t in input_tokens_batched]
        if sum(q_lens) != num_tokens:
            raise ValueError(f"num_tokens {num_tokens} != {sum(q_lens)} input tokens")
        if not 0 <= local_layer_start < local_layer_end <= self.layers:
            raise ValueError("local layer range outside the model")
        if num_restore_requests:
            raise NotImplementedError("live KV restore inside pforward is not part of this path")
        stage_layers = local_layer_end - local_layer_start
        if stage_layers == self.layers:
            pool, id_map, num_ids, offset = self.pool, None, self.max_num_pages, 0
        else:
            if self.layers % stage_layers or local_layer_start % stage_layers:
                raise ValueError(f"layers [{local_layer_start}, {local_layer_end}) are not one "
                                 f"of {self.layers} // {stage_layers} equal pipeline stages")
            n = self.layers // stage_layers
            pool = self.fused_pool(n)
            num_ids = pool.num_pages
            base = self.num_base_pages

            def id_map(ids, base=base, n=n, num_ids=num_ids):
                return fused_page_ids(ids, base, n, num_ids)
            offset = local_layer_start
        if max_num_pages > num_ids:
            raise ValueError(f"max_num_pages {max_num_pages} exceeds the pool "
                             f"({num_ids} pages in this id space)")
        step = AttentionStep(pool, self.qo_head, q_lens, first_token_indexes,
                             is_prefill_requests, pages_of_reqs,
                             use_tensor_cores=self.use_tensor_cores,
                             is_context_stage=is_context_stage, layer_offset=offset,
                             id_map=id_map, num_ids=min(max_num_pages, num_ids))
        step.layer_range = (local_layer_start, local_layer_end)
        return step

    def fused_pool(self, fusion_size: int) -> KVPool:
        """The pool in the fused page-id space of a group of fusion_size
        instances (see the module docstring); fusion_size 1 is the pool."""
        if fusion_size == 1:
            return self.pool
        return self.pool.fused_view(self.num_base_pages, fusion_size)

    def num_fused_pages(self, fusion_size: int) -> int:
        """P * N + E: the fused ids the block manager may hand out."""
        return self.max_num_pages * fusion_size

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
        """Joins a balloon group of num_group_instances instances as stage
        rank_in_group: drops the weights of every layer outside the stage and
        returns the number of KV blocks they became (kunserve/worker.py:454-458).
        Blocks are counted as the fused stage uses them, G = layers /
        num_group_instances layers each, and are the fused extend ids
        [P*N, P*N + returned) (add_ex_fusion_blocks,
        kunserve/block_manager.py:262-269), in order of the dropped layers.
        K takes the first half of each layer's memory and V the second. Waits
        for the device. Views of the dropped weights must not be used
        afterwards. Without max_extend_pages nothing can be dropped and 0 is
        returned."""
        keep = kept_layers(self.layers, rank_in_group, num_group_instances)
        self.fusion_size = num_group_instances
        if self.pmm is None:
            return 0
        dropped = set(self.dropped_layers())
        added = 0
        for layer in sorted(self._weight_segments):
            if layer in keep or layer in dropped:
                continue
            added += len(self.pmm.drop(self._weight_segments[layer]))
        self._sync_pool()
        return added * num_group_instances

    def pmm_restore(self) -> List[int]:
        """Maps every dropped layer's memory back to its weights and returns
        those layers (kunserve/worker.py:484-487); their blocks leave the
        pool, so no request may hold them. The memory comes back holding KV
        data: the weights themselves are reloaded by the caller (the
        reference pulls them from a peer instance over NCCL,
        kunserve/llm_engine.py:553-558). The op leaves its balloon group:
        page ids are unfused again (restore_from_fusion resets the fusion
        size, kunserve/block_manager.py:347-348). Without max_extend_pages
        nothing was dropped and [] is returned."""
        self.fusion_size = 1
        if self.pmm is None:
            return []
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
        """Copies extend-region blocks into base-region blocks, all layers of
        a block (kunserve/worker.py:818-823; caller
        kunserve/flash_backend.py:1116-1123). In a balloon group (after
        pmm_drop with N > 1) max_num_pages = P*N + E names the fused id space
        (kunserve/flash_backend.py:2435-2440) and a block is a fused page of
        layers / N layers; otherwise ids name whole pages."""
        if len(all_ex_blocks) != len(all_base_blocks):
            raise ValueError("ex and base block lists differ in length")
        fused = self.fusion_size > 1 and max_num_pages > self.max_num_pages
        limit = min(max_num_pages, self.num_fused_pages(self.fusion_size) if fused
                    else self.max_num_pages)
        ids = np.asarray(list(all_ex_blocks) + list(all_base_blocks), dtype=np.int64)
        if ids.size and (ids.min() < 0 or ids.max() >= limit):
            raise IndexError(f"block id outside [0, {limit})")
        if len(set(all_ex_blocks) & set(all_base_blocks)):
            raise ValueError("source and destination blocks overlap")
        if not fused:
            copy_blocks(self.pool, all_ex_blocks, all_base_blocks)
            return
        pool = self.fused_pool(self.fusion_size)
        n = self.fusion_size
        copy_blocks(pool, fused_page_ids(all_ex_blocks, self.num_base_pages, n, pool.num_pages),
                    fused_page_ids(all_base_blocks, self.num_base_pages, n, pool.num_pages))

    def kv_exchange_pack(self, page_ids: Sequence[int], layer_begin: int, layer_end: int,
                         scratch: Optional[torch.Tensor] = None) -> torch.Tensor:
        """kv_exchange phase 1: gathers the sender's pages (sorted pre-fusion
        local ids, kunserve/flash_backend.py:913-928) for layers
        [layer_begin, layer_end) into one contiguous buffer."""
        return kv_pack(self.pool, layer_begin, layer_end, page_ids, scratch)

    def kv_exchange_scatter(self, page_ids: Sequence[int], layer_begin: int, layer_end: int,
                            scratch: torch.Tensor) -> None:
        """kv_exchange phase 3: writes received pages into this instance's
        fused page ids (kunserve/block_manager.py:755-763). Layers
        [layer_begin, layer_end) are model layers of this instance's stage in
        its balloon group (pmm_drop); they land in the fused pages' G-layer
        slabs. Outside a group the ids are whole pages."""
        n = self.fusion_size
        if n == 1:
            kv_scatter(self.pool, layer_begin, layer_end, page_ids, scratch)
            return
        g = self.layers // n
        stage = layer_begin // g
        if not (0 <= layer_begin < layer_end <= (stage + 1) * g):
            raise ValueError(f"layers [{layer_begin}, {layer_end}) are not within one stage "
                             f"of {g} layers")
        pool = self.fused_pool(n)
        ids = fused_page_ids(page_ids, self.num_base_pages, n, pool.num_pages)
        kv_scatter(pool, layer_begin - stage * g, layer_end - stage * g, ids, scratch)

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
