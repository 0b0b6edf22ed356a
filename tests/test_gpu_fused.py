"""The fused page-id space of a balloon group on the GPU
(kunserve/block_manager.py:231-281, kunserve/flash_backend.py:709-725,2433-2445).

After pmm_drop(rank, N) an instance runs one pipeline stage of G = L / N
layers and its block manager hands out fused ids: i*P + b is layer group i
of base page b, ids from P*N on are extend pages of G layers. pforward over
the stage must
  * read the stale requests' kept ids r*P + b in place: bit-exact equal to
    the same step over page b before the fusion;
  * append, decode and prefill over a table mixing fused base and extend ids
    as the oracle does on the pool seen through its fused address map
    (oracle.fused_pool_copy, built slab by slab from fused_slab);
and local_copy_blocks and the kv_exchange scatter must move G-layer fused
pages, bit-exact."""
import math

import numpy as np
import pytest
import torch

from kunserve_amd import LlamaOp
from oracle import paged_attention_ref as ref

from helpers import ATOL, max_abs, random_tensor, to_numpy

pytestmark = pytest.mark.gpu


def fill(op, seed):
    g = torch.Generator(device=op.pool.device)
    g.manual_seed(seed)
    for t in (op.pool.k, op.pool.v):
        t.copy_(torch.randn(t.shape, generator=g, device=t.device).to(t.dtype))


def step_inputs(T, hq, hkv, device, seed):
    return (random_tensor((T, hq, 128), device, seed), random_tensor((T, hkv, 128), device, seed + 1),
            random_tensor((T, hkv, 128), device, seed + 2))


@pytest.mark.parametrize("hq,hkv", [(8, 8), (8, 2), (16, 2)])
def test_kept_ids_read_the_prefusion_pages_bit_exact(device, hq, hkv):
    """Stage r of a 2-instance group over kept ids r*P + b equals the
    unfused step over pages b at the same model layers, bit for bit: the
    append, decode (VALU for 1 q head per KV head, MFMA for 4 and 8) and
    prefill."""
    P, L, N = 48, 4, 2
    op = LlamaOp(P, L, hq, hkv, 16, 128, 1, 1, 8, 4096, 4096, 1, device)
    fill(op, 1)
    rng = np.random.default_rng(2)
    first, flags, q_lens = [200, 31, 0, 90], [0, 1, 1, 0], [1, 40, 17, 1]
    kv = ref.kv_lens_for_step(first, q_lens, flags)
    need = (kv + 15) // 16
    perm = rng.permutation(P)
    pages, at = [], 0
    for n in need:
        pages.append(perm[at:at + n].tolist())
        at += n
    T = sum(q_lens)
    q, k, v = step_inputs(T, hq, hkv, device, 10)
    tokens = [[0] * n for n in q_lens]
    k0, v0 = op.pool.k.clone(), op.pool.v.clone()

    unfused = op.pforward(4, T, P, 0, L, tokens, first, flags, pages)
    out_a = [unfused.run(layer, q.clone(), k, v) for layer in (2, 3)]
    ka, va = op.pool.k.clone(), op.pool.v.clone()

    op.pool.k.copy_(k0)
    op.pool.v.copy_(v0)
    r = 1
    assert op.pmm_drop(r, N) == 0                     # no weight memory to drop here
    kept = [[ref.kept_page_id(b, P * N, N, r) for b in row] for row in pages]
    fused = op.pforward(4, T, P * N, 2, 4, tokens, first, flags, kept)
    out_b = [fused.run(layer, q.clone(), k, v) for layer in (2, 3)]
    torch.cuda.synchronize()
    for a, b in zip(out_a, out_b):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.equal(op.pool.k.view(torch.int16), ka.view(torch.int16))
    assert torch.equal(op.pool.v.view(torch.int16), va.view(torch.int16))
    with pytest.raises(ValueError, match="pipeline stages"):
        op.pforward(4, T, P * N, 1, 3, tokens, first, flags, kept)


def test_fused_and_extend_table_matches_oracle(device):
    """A 4-layer model in a 2-instance group, stage 0, after pmm_drop turned
    layers 2 and 3 into extend pages: rows mix fused base ids of both layer
    groups with extend ids. Append bit-exact and attention within ATOL of
    the oracle run on the fused pool copy."""
    P, L, N, hq, hkv = 24, 4, 2, 8, 2
    op = LlamaOp(P, L, hq, hkv, 16, 128, 1, 1, 8, 4096, 4096, 1, device=device,
                 max_extend_pages=16)
    pb = op.pmm.page_bytes
    for layer in range(L):
        op.layer_weights(layer, 3 * pb)              # 2 page pairs per layer
    E = op.pmm_drop(0, N)
    assert E == 2 * 2 * N                            # 2 layers x 2 pages x N fused pages
    assert op.max_num_pages == P + 4 and op.num_fused_pages(N) == P * N + E
    fill(op, 3)
    rng = np.random.default_rng(4)
    ids = rng.permutation(P * N + E)
    first, flags, q_lens = [130, 0, 61, 300], [0, 1, 1, 0], [1, 70, 33, 1]
    kv = ref.kv_lens_for_step(first, q_lens, flags)
    need = (kv + 15) // 16
    pages, at = [], 0
    for n in need:
        pages.append(ids[at:at + n].tolist())
        at += n
    flat = np.concatenate(pages)
    assert (flat >= P * N).any() and (flat < P).any() and ((flat >= P) & (flat < P * N)).any()
    T = sum(q_lens)
    q, k, v = step_inputs(T, hq, hkv, device, 20)
    fk = ref.fused_pool_copy(to_numpy(op.pool.k), P, N)
    fv = ref.fused_pool_copy(to_numpy(op.pool.v), P, N)
    step = op.pforward(4, T, P * N + E, 0, 2, [[0] * n for n in q_lens], first, flags, pages)
    out = step.run(1, q, k, v)
    torch.cuda.synchronize()
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)])
    indptr = np.concatenate([[0], np.cumsum(need)])
    ref.append_kv(fk, fv, 1, indptr, flat, kv, q_indptr, to_numpy(k), to_numpy(v))
    assert np.array_equal(ref.fused_pool_copy(to_numpy(op.pool.k), P, N).view(np.int16),
                          fk.view(np.int16))
    assert np.array_equal(ref.fused_pool_copy(to_numpy(op.pool.v), P, N).view(np.int16),
                          fv.view(np.int16))
    want = ref.prefill_attention(to_numpy(q), q_indptr, fk, fv, 1, indptr, flat, kv,
                                 1 / math.sqrt(128))
    assert max_abs(out, want) <= ATOL
    with pytest.raises(ValueError, match="exceeds"):
        op.pforward(4, T, P * N + E + 1, 0, 2, [[0] * n for n in q_lens], first, flags, pages)
    with pytest.raises(IndexError):
        op.pforward(4, T, P * N + E, 0, 2, [[0] * n for n in q_lens], first, flags,
                    [[P * N + E] + pages[0][1:]] + pages[1:])
    op.pmm_restore()
    # after the restore the fused base ids stay valid for the group's requests
    # (kunserve/flash_backend.py:2436-2438), the extend ids are gone
    assert op.num_fused_pages(N) == P * N
    op.pmm.close()


def test_fused_local_copy_blocks(device):
    """local_copy_blocks in the fused space (max_num_pages = P*N + E) moves
    G-layer fused pages: extend ids into base ids, nothing else changes."""
    P, L, N = 16, 4, 2
    op = LlamaOp(P, L, 4, 4, 16, 128, 1, 1, 8, 4096, 4096, 1, device=device,
                 max_extend_pages=8)
    for layer in range(L):
        op.layer_weights(layer, 2 * op.pmm.page_bytes)
    E = op.pmm_drop(1, N)
    fill(op, 5)
    before_k = ref.fused_pool_copy(to_numpy(op.pool.k), P, N)
    before_v = ref.fused_pool_copy(to_numpy(op.pool.v), P, N)
    ex = [P * N + 0, P * N + 2, P * N + E - 1]
    base = [5, P + 2, 2 * P - 1]                    # both layer groups of the base pages
    op.local_copy_blocks(P * N + E, ex, base)
    torch.cuda.synchronize()
    after_k = ref.fused_pool_copy(to_numpy(op.pool.k), P, N)
    after_v = ref.fused_pool_copy(to_numpy(op.pool.v), P, N)
    want_k, want_v = before_k.copy(), before_v.copy()
    want_k[base], want_v[base] = before_k[ex], before_v[ex]
    assert np.array_equal(after_k.view(np.int16), want_k.view(np.int16))
    assert np.array_equal(after_v.view(np.int16), want_v.view(np.int16))
    with pytest.raises(IndexError):
        op.local_copy_blocks(P * N + E, [P * N + E], [0])
    op.pmm.close()


def test_exchange_into_fused_ids_then_decode(device):
    """kv_exchange's single-GPU halves between two instances of a 2-instance
    group: instance 0 packs stale pages (pre-fusion ids) for stage 1's
    layers, instance 1 scatters them into fused ids it allocated; decode of
    stage 1 over those ids then equals instance 0's decode over the
    original pages, bit for bit."""
    P, L, N, hq, hkv = 32, 4, 2, 8, 2
    a = LlamaOp(P, L, hq, hkv, 16, 128, 1, 1, 8, 4096, 4096, 1, device)
    b = LlamaOp(P, L, hq, hkv, 16, 128, 1, 1, 8, 4096, 4096, 1, device)
    fill(a, 7)
    fill(b, 8)
    b.pmm_drop(1, N)
    src = sorted([9, 2, 13, 27, 4])
    dst = [ref.fused_page_ids(p, P, N)[0] for p in (3, 30, 11, 7, 19)]   # layer group 0 pages
    scr = a.kv_exchange_pack(src, 2, 4)
    b.kv_exchange_scatter(dst, 2, 4, scr)
    # one decode row over the 5 pages (80 tokens), no new token appended
    # before attention reads: compare the stage's layers 2 and 3
    first, flags, q_lens = [80], [0], [1]
    q, k, v = step_inputs(1, hq, hkv, device, 30)
    step_a = a.pforward(1, 1, P, 0, L, [[0]], first, flags, [src])
    step_b = b.pforward(1, 1, P * N, 2, 4, [[0]], first, flags, [dst])
    for layer in (2, 3):
        oa = step_a.run(layer, q.clone(), k, v)
        ob = step_b.run(layer, q.clone(), k, v)
        torch.cuda.synchronize()
        assert torch.equal(oa.view(torch.int16), ob.view(torch.int16))
    with pytest.raises(ValueError, match="one stage"):
        b.kv_exchange_scatter(dst, 1, 3, scr)
