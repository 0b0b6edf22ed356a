"""Parameter memory remap (pmm_drop / pmm_restore, kunserve/worker.py:454-501)
on the GPU.

Dropping a weight segment must make its bytes the K and V pages numbered
after the current ones (kunserve/block_manager.py:262-269), leave every
existing page and every kept weight untouched, and restoring must give the
segment back holding what those pages held: all bit-exact. Attention, the
K/V append and block copies over extend pages are checked against the oracle
(max-abs <= ATOL for attention, bit-exact for the byte movers)."""
import math

import numpy as np
import pytest
import torch

from kunserve_amd import AttentionStep, LlamaOp, PmmPool, copy_blocks
from kunserve_amd._lib import KunserveError
from oracle import paged_attention_ref as ref

from helpers import ATOL, max_abs, random_tensor

pytestmark = pytest.mark.gpu


def bytes_of(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous().view(torch.uint8).reshape(t.shape[0], -1)


def random_bytes(n, device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return torch.randint(0, 256, (n,), generator=g, device=device, dtype=torch.uint8)


def test_drop_and_restore_move_segment_bytes(device):
    pm = PmmPool(8, 2, 2, 16, 128, 12, device)
    try:
        assert pm.page_bytes == 2 * 2 * 16 * 128 * 2 and pm.num_pages == 8
        pool = pm.pool
        pool.k.copy_(random_tensor(pool.k.shape, device, 1))
        pool.v.copy_(random_tensor(pool.v.shape, device, 2))
        k0, v0 = bytes_of(pool.k).clone(), bytes_of(pool.v).clone()
        s0 = pm.add_segment(3 * 2 * pm.page_bytes)
        s1 = pm.add_segment(1)                       # rounds up to one page pair
        assert pm.segment_pages(s0) == 3 and pm.segment_pages(s1) == 1
        b0 = random_bytes(3 * 2 * pm.page_bytes, device, 3)
        b1 = random_bytes(2 * pm.page_bytes, device, 4)
        pm.segment(s0).copy_(b0)
        pm.segment(s1).copy_(b1)
        torch.cuda.synchronize()

        old = pm.pool
        assert pm.drop(s0) == range(8, 11)
        with pytest.raises(RuntimeError, match="predates"):
            copy_blocks(old, [0], [1])
        with pytest.raises(RuntimeError, match="dropped"):
            pm.segment(s0)
        kb, vb = bytes_of(pm.pool.k), bytes_of(pm.pool.v)
        half = 3 * pm.page_bytes
        assert torch.equal(kb[8:11].flatten(), b0[:half])
        assert torch.equal(vb[8:11].flatten(), b0[half:])
        assert torch.equal(kb[:8], k0) and torch.equal(vb[:8], v0)

        assert pm.drop(s1) == range(11, 12)
        kb, vb = bytes_of(pm.pool.k), bytes_of(pm.pool.v)
        assert torch.equal(kb[11], b1[:pm.page_bytes]) and torch.equal(vb[11], b1[pm.page_bytes:])
        assert torch.equal(kb[8:11].flatten(), b0[:half])

        # a drop beyond the reserved extend pages fails and changes nothing
        big = pm.add_segment(9 * 2 * pm.page_bytes)   # 8 extend pages are left
        with pytest.raises(KunserveError, match="extend pages"):
            pm.drop(big)
        assert pm.num_pages == 12 and pm.dropped == [s0, s1]
        with pytest.raises(KunserveError, match="already dropped"):
            pm.drop(s0)

        # pages written while extended travel back with the segment
        pm.pool.k[11].fill_(1.5)
        pm.pool.v[9].fill_(-2.0)
        torch.cuda.synchronize()
        k9 = bytes_of(pm.pool.k)[8:11].flatten().clone()
        v9 = bytes_of(pm.pool.v)[8:11].flatten().clone()
        v11 = bytes_of(pm.pool.v)[11].clone()
        assert pm.restore() == s1 and pm.num_pages == 11
        seg1 = pm.segment(s1)
        assert torch.equal(seg1[:pm.page_bytes].view(torch.float16),
                           torch.full((pm.page_elems,), 1.5, device=device, dtype=torch.float16))
        assert torch.equal(seg1[pm.page_bytes:], v11)
        assert pm.restore() == s0 and pm.num_pages == 8
        seg0 = pm.segment(s0)
        assert torch.equal(seg0[:half], k9) and torch.equal(seg0[half:], v9)
        assert torch.equal(bytes_of(pm.pool.k), k0) and torch.equal(bytes_of(pm.pool.v), v0)
        with pytest.raises(KunserveError, match="no dropped segment"):
            pm.restore()

        # the big segment drops now that there is room, and the pages follow
        assert pm.drop(big) == range(8, 17)
        assert pm.restore() == big
    finally:
        pm.close()


def test_attention_and_copies_on_extend_pages(device):
    """A pforward step whose rows mix base pages and pages of a dropped
    segment, then copies from extend blocks into base blocks
    (LlamaOp.local_copy_blocks, kunserve/flash_backend.py:1116-1123)."""
    hq, hkv, ps, d, layers = 8, 2, 16, 128, 2
    pm = PmmPool(16, layers, hkv, ps, d, 16, device)
    try:
        pool = pm.pool
        pool.k.copy_(random_tensor(pool.k.shape, device, 5))
        pool.v.copy_(random_tensor(pool.v.shape, device, 6))
        sid = pm.add_segment(8 * 2 * pm.page_bytes)
        pm.segment(sid).view(torch.float16).copy_(
            random_tensor((8 * 2 * pm.page_elems,), device, 7))
        assert pm.drop(sid) == range(16, 24)
        pool = pm.pool
        pages = [[17, 3, 22], [20, 5, 16, 19, 23]]
        q_lens, first, flags = [1, 45], [40, 20], [0, 1]
        step = AttentionStep(pool, hq, q_lens, first, flags, pages)
        T = sum(q_lens)
        q = random_tensor((T, hq, d), device, 8)
        k = random_tensor((T, hkv, d), device, 9)
        v = random_tensor((T, hkv, d), device, 10)
        kh, vh = pool.k.cpu().numpy(), pool.v.cpu().numpy()
        out = step.run(1, q, k, v)
        torch.cuda.synchronize()
        kv = np.array([40, 65])
        q_indptr = np.array([0, 1, 46])
        indptr, indices = step.table.indptr_host, step.table.indices_host
        ref.append_kv(kh, vh, 1, indptr, indices, kv, q_indptr, k.cpu().numpy(),
                      v.cpu().numpy())
        assert np.array_equal(pool.k.cpu().numpy().view(np.int16), kh.view(np.int16))
        assert np.array_equal(pool.v.cpu().numpy().view(np.int16), vh.view(np.int16))
        want = ref.prefill_attention(q.cpu().numpy(), q_indptr, kh, vh, 1, indptr, indices, kv,
                                     1 / math.sqrt(d))
        assert max_abs(out, want) <= ATOL

        copy_blocks(pool, [17, 20, 23], [2, 9, 15])
        torch.cuda.synchronize()
        kb, vb = bytes_of(pool.k), bytes_of(pool.v)
        assert torch.equal(kb[[2, 9, 15]], kb[[17, 20, 23]])
        assert torch.equal(vb[[2, 9, 15]], vb[[17, 20, 23]])
    finally:
        pm.close()


def test_llama_op_pmm_drop_and_restore(device):
    """LlamaOp.pmm_drop(rank, group) drops the layers outside the rank's stage
    and returns the block count (kunserve/worker.py:454-458); the blocks are
    num_base + k; pmm_restore gives the layers back."""
    layers, base = 4, 16
    op = LlamaOp(base, layers, 8, 2, 16, 128, 11008, 32000, 8, 4096, 4096, 1, device=device,
                 max_extend_pages=64)
    pb = op.pmm.page_bytes
    assert pb == layers * 2 * 16 * 128 * 2
    nbytes = 3 * pb + 100                     # rounds up to 2 page pairs per layer
    w = [op.layer_weights(layer, nbytes) for layer in range(layers)]
    for layer, t in enumerate(w):
        t.copy_(random_bytes(t.numel(), device, 20 + layer))
    host = [t.cpu() for t in w]
    del w
    g = torch.Generator(device=device)
    g.manual_seed(30)
    for t in (op.pool.k, op.pool.v):
        t.copy_(torch.randn(t.shape, generator=g, device=device).half())

    # layers 2 and 3, 2 blocks each, counted as the 2-layer blocks of the fused stage
    assert op.pmm_drop(0, 2) == 8
    assert op.dropped_layers() == [2, 3] and op.max_num_pages == base + 4
    assert op.num_fused_pages(2) == 2 * base + 8
    kb, vb = bytes_of(op.pool.k), bytes_of(op.pool.v)
    for i, layer in enumerate((2, 3)):
        ids = slice(base + 2 * i, base + 2 * i + 2)
        assert torch.equal(kb[ids].flatten().cpu(), host[layer][:2 * pb])
        assert torch.equal(vb[ids].flatten().cpu(), host[layer][2 * pb:])
    for layer in (0, 1):
        assert torch.equal(op.layer_weights(layer, nbytes).cpu(), host[layer])
    assert op.pmm_drop(0, 2) == 0             # nothing left to drop for this stage

    # the extend blocks hold weight bytes, not numbers: overwrite them with
    # values first, as the engine's appends would
    op.pool.k[base:].copy_(torch.randn(op.pool.k[base:].shape, generator=g,
                                       device=device).half())
    op.pool.v[base:].copy_(torch.randn(op.pool.v[base:].shape, generator=g,
                                       device=device).half())
    # stage 0 of the group runs layers [0, 2) over fused ids: extend ids from 2 * base
    fused_ext = 2 * base
    q_lens, first, flags = [1, 20], [30, 12], [0, 1]
    pages = [[fused_ext + 1, 4], [fused_ext + 7, fused_ext + 2]]
    step = op.pforward(2, 21, op.num_fused_pages(2), 0, 2, [[0] * n for n in q_lens], first,
                       flags, pages)
    q = random_tensor((21, 8, 128), device, 31)
    k = random_tensor((21, 2, 128), device, 32)
    v = random_tensor((21, 2, 128), device, 33)
    kh = ref.fused_pool_copy(op.pool.k.cpu().numpy(), base, 2)
    vh = ref.fused_pool_copy(op.pool.v.cpu().numpy(), base, 2)
    out = step.run(0, q, k, v)
    torch.cuda.synchronize()
    kv = np.array([30, 32])
    q_indptr = np.array([0, 1, 21])
    indptr = np.array([0, 2, 4])
    indices = np.array([fused_ext + 1, 4, fused_ext + 7, fused_ext + 2])
    ref.append_kv(kh, vh, 0, indptr, indices, kv, q_indptr, k.cpu().numpy(), v.cpu().numpy())
    assert np.array_equal(ref.fused_pool_copy(op.pool.k.cpu().numpy(), base, 2).view(np.int16),
                          kh.view(np.int16))
    want = ref.prefill_attention(q.cpu().numpy(), q_indptr, kh, vh, 0, indptr, indices, kv,
                                 1 / math.sqrt(128))
    assert max_abs(out, want) <= ATOL

    k_ext = bytes_of(op.pool.k)[base + 2:base + 4].flatten().cpu()
    assert op.pmm_restore() == [2, 3]
    assert op.dropped_layers() == [] and op.max_num_pages == base
    assert torch.equal(op.layer_weights(3, nbytes)[:2 * pb].cpu(), k_ext)
    for layer in (0, 1):
        assert torch.equal(op.layer_weights(layer, nbytes).cpu(), host[layer])
    with pytest.raises(ValueError, match="exceeds the pool"):
        op.pforward(2, 21, 2 * base + 8, 0, 2, [[0] * n for n in q_lens], first, flags, pages)
    with pytest.raises(IndexError):
        op.pforward(2, 21, 2 * base, 0, 2, [[0] * n for n in q_lens], first, flags, pages)
    # the restore leaves the group: kv_exchange_scatter takes unfused ids
    # again, whole pages of all layers (block_manager.py:347-348)
    assert op.fusion_size == 1
    before_k, before_v = op.pool.k.clone(), op.pool.v.clone()
    packed = op.kv_exchange_pack([3, 9], 1, 4)
    op.kv_exchange_scatter([5, 12], 1, 4, packed)
    torch.cuda.synchronize()
    want_k, want_v = before_k.clone(), before_v.clone()
    want_k[[5, 12], 1:4] = before_k[[3, 9], 1:4]
    want_v[[5, 12], 1:4] = before_v[[3, 9], 1:4]
    assert torch.equal(op.pool.k.view(torch.int16), want_k.view(torch.int16))
    assert torch.equal(op.pool.v.view(torch.int16), want_v.view(torch.int16))
    op.pmm.close()
