"""Pins the CPU oracle (oracle/paged_attention_ref.py) before it is trusted.

Each check is chosen so that a plausible slip in the oracle (slot vs page
index swapped, wrong scale, GQA head mapping h % Hkv instead of h // G, an
off-by-one in the causal bound or in the first-index rule) fails one of
them. The attention references are torch's scaled_dot_product_attention in
float64 on dense K/V; the dense K/V are written into pages by a separate
element loop, not by the oracle's gather.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import paged_attention_ref as ref

from lifecycle import Request


def scatter_dense(dense_k, dense_v, num_pages, num_layers, layer, page_size, rng):
    """Writes per-sequence dense K/V [Hkv, n, D] into random pages with an
    explicit element loop; returns pools and CSR tables."""
    hkv, d = dense_k[0].shape[0], dense_k[0].shape[2]
    kp = rng.standard_normal((num_pages, num_layers, hkv, page_size, d))
    vp = rng.standard_normal((num_pages, num_layers, hkv, page_size, d))
    perm = rng.permutation(num_pages)
    indptr, indices, at = [0], [], 0
    for K, V in zip(dense_k, dense_v):
        n = K.shape[1]
        npg = (n + page_size - 1) // page_size
        pages = perm[at:at + npg]
        at += npg
        for t in range(n):
            page, slot = pages[t // page_size], t % page_size
            for h in range(hkv):
                kp[page, layer, h, slot, :] = K[h, t]
                vp[page, layer, h, slot, :] = V[h, t]
        indices.extend(pages.tolist())
        indptr.append(len(indices))
    return kp, vp, np.array(indptr), np.array(indices)


def sdpa(q, k, v, causal=False, scale=None):
    return F.scaled_dot_product_attention(torch.from_numpy(q), torch.from_numpy(k),
                                          torch.from_numpy(v), is_causal=causal,
                                          scale=scale).numpy()


@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 2)])
def test_decode_matches_sdpa_on_dense(hq, hkv):
    rng = np.random.default_rng(0)
    d, ps, L, layer = 32, 4, 3, 1
    lens = [1, 5, 13, 16]
    dk = [rng.standard_normal((hkv, n, d)) for n in lens]
    dv = [rng.standard_normal((hkv, n, d)) for n in lens]
    kp, vp, indptr, indices = scatter_dense(dk, dv, 32, L, layer, ps, rng)
    q = rng.standard_normal((len(lens), hq, d))
    scale = 1 / math.sqrt(d)
    out = ref.decode_attention(q, kp, vp, layer, indptr, indices, np.array(lens), scale)
    g = hq // hkv
    for b, n in enumerate(lens):
        K = np.repeat(dk[b], g, axis=0)   # head h uses kv head h // g
        V = np.repeat(dv[b], g, axis=0)
        want = sdpa(q[b][:, None, :], K, V, scale=scale)[:, 0]
        np.testing.assert_allclose(out[b], want, rtol=1e-12, atol=1e-12)


def test_decode_closed_forms():
    rng = np.random.default_rng(1)
    d, ps, hkv = 16, 4, 2
    lens = [1, 9]
    dk = [rng.standard_normal((hkv, n, d)) for n in lens]
    dv = [rng.standard_normal((hkv, n, d)) for n in lens]
    kp, vp, indptr, indices = scatter_dense(dk, dv, 8, 1, 0, ps, rng)
    q = rng.standard_normal((2, hkv, d))
    out = ref.decode_attention(q, kp, vp, 0, indptr, indices, np.array(lens), 0.3)
    # kv_len 1: the output is that token's V.
    np.testing.assert_allclose(out[0], dv[0][:, 0], rtol=0, atol=1e-15)
    # q = 0: uniform weights, the output is the mean of V.
    out0 = ref.decode_attention(np.zeros_like(q), kp, vp, 0, indptr, indices, np.array(lens), 0.3)
    np.testing.assert_allclose(out0[1], dv[1].mean(axis=1), rtol=1e-13, atol=1e-13)
    # kv_len 0 yields zeros.
    z = ref.decode_attention(q[:1], kp, vp, 0, np.array([0, 0]), np.array([], dtype=int),
                             np.array([0]), 0.3)
    assert np.all(z == 0)


def test_decode_page_permutation_invariance():
    rng = np.random.default_rng(2)
    d, ps, hkv, npg = 8, 4, 2, 16
    kp = rng.standard_normal((npg, 1, hkv, ps, d))
    vp = rng.standard_normal((npg, 1, hkv, ps, d))
    indptr = np.array([0, 3, 7])
    indices = rng.permutation(npg)[:7]
    kv = np.array([10, 14])
    q = rng.standard_normal((2, hkv, d))
    base = ref.decode_attention(q, kp, vp, 0, indptr, indices, kv, 0.5)
    perm = rng.permutation(npg)             # physical page p moves to perm[p]
    kp2, vp2 = np.empty_like(kp), np.empty_like(vp)
    kp2[perm], vp2[perm] = kp, vp
    moved = ref.decode_attention(q, kp2, vp2, 0, indptr, perm[indices], kv, 0.5)
    np.testing.assert_allclose(moved, base, rtol=0, atol=1e-15)


def test_gqa_equals_repeated_mha():
    rng = np.random.default_rng(3)
    d, ps, hkv, g, npg = 8, 4, 2, 4, 12
    kp = rng.standard_normal((npg, 1, hkv, ps, d))
    vp = rng.standard_normal((npg, 1, hkv, ps, d))
    indptr, indices, kv = np.array([0, 5]), rng.permutation(npg)[:5], np.array([18])
    q = rng.standard_normal((1, hkv * g, d))
    gqa = ref.decode_attention(q, kp, vp, 0, indptr, indices, kv, 0.4)
    mha = ref.decode_attention(q, np.repeat(kp, g, axis=2), np.repeat(vp, g, axis=2), 0, indptr,
                               indices, kv, 0.4)
    np.testing.assert_allclose(gqa, mha, rtol=0, atol=1e-15)


def test_prefill_without_prefix_matches_causal_sdpa():
    rng = np.random.default_rng(4)
    d, ps, h = 16, 4, 3
    lens = [7, 12]
    dk = [rng.standard_normal((h, n, d)) for n in lens]
    dv = [rng.standard_normal((h, n, d)) for n in lens]
    kp, vp, indptr, indices = scatter_dense(dk, dv, 16, 2, 1, ps, rng)
    q_indptr = np.array([0, 7, 19])
    q = rng.standard_normal((19, h, d))
    out = ref.prefill_attention(q, q_indptr, kp, vp, 1, indptr, indices, np.array(lens), 0.25)
    for b, n in enumerate(lens):
        qb = q[q_indptr[b]:q_indptr[b + 1]].transpose(1, 0, 2)
        want = sdpa(qb, dk[b], dv[b], causal=True, scale=0.25).transpose(1, 0, 2)
        np.testing.assert_allclose(out[q_indptr[b]:q_indptr[b + 1]], want, rtol=1e-12,
                                   atol=1e-12)


def test_prefill_row_equals_decode_over_its_prefix():
    rng = np.random.default_rng(5)
    d, ps, hkv, g, npg = 8, 4, 2, 2, 20
    kp = rng.standard_normal((npg, 1, hkv, ps, d))
    vp = rng.standard_normal((npg, 1, hkv, ps, d))
    indices = rng.permutation(npg)[:6]
    kv, ql = 23, 5                    # prefix 18 cached, 5 new rows
    q = rng.standard_normal((ql, hkv * g, d))
    out = ref.prefill_attention(q, np.array([0, ql]), kp, vp, 0, np.array([0, 6]), indices,
                                np.array([kv]), 0.3)
    for i in range(ql):
        dec = ref.decode_attention(q[i:i + 1], kp, vp, 0, np.array([0, 6]), indices,
                                   np.array([kv - ql + i + 1]), 0.3)
        np.testing.assert_allclose(out[i], dec[0], rtol=0, atol=1e-14)


def _unique_pool(shape):
    """int16 pool whose every element is distinct (mod 2^16), so a misplaced
    element is visible."""
    return (np.arange(np.prod(shape), dtype=np.int64) % 65521).astype(np.int16).reshape(shape)


def test_append_matches_element_loop():
    rng = np.random.default_rng(6)
    npg, L, hkv, ps, d = 10, 2, 2, 4, 3
    kp, vp = _unique_pool((npg, L, hkv, ps, d)), -_unique_pool((npg, L, hkv, ps, d))
    indptr, indices = np.array([0, 3, 5]), np.array([7, 2, 9, 0, 4])
    kv, q_indptr = np.array([10, 6]), np.array([0, 4, 5])
    kn = rng.integers(-999, 999, (5, hkv, d)).astype(np.int16)
    vn = rng.integers(-999, 999, (5, hkv, d)).astype(np.int16)
    k1, v1 = kp.copy(), vp.copy()
    ref.append_kv(k1, v1, 1, indptr, indices, kv, q_indptr, kn, vn)
    k2, v2 = kp.copy(), vp.copy()
    # row 0: positions 6..9 -> pages 2 (slots 2,3) and 9 (slots 0,1); row 1: position 5 -> page 4 slot 1
    for tok, (page, slot) in enumerate([(2, 2), (2, 3), (9, 0), (9, 1), (4, 1)]):
        for h in range(hkv):
            for e in range(d):
                k2[page, 1, h, slot, e] = kn[tok, h, e]
                v2[page, 1, h, slot, e] = vn[tok, h, e]
    assert np.array_equal(k1, k2) and np.array_equal(v1, v2)


def test_copy_swap_pack_scatter_match_element_loops():
    shape = (12, 2, 2, 4, 3)
    pool = _unique_pool(shape)
    src, dst = [1, 5, 6], [9, 0, 11]
    got = pool.copy()
    ref.copy_blocks(got, src, dst)
    want = pool.copy()
    for s, t in zip(src, dst):
        for idx in np.ndindex(shape[1:]):
            want[(t,) + idx] = pool[(s,) + idx]
    assert np.array_equal(got, want)

    host = np.zeros((4,) + shape[1:], dtype=np.int16)
    ref.swap([3, 7], [2, 0], pool, host)
    assert np.array_equal(host[2], pool[3]) and np.array_equal(host[0], pool[7])
    assert not host[1].any() and not host[3].any()

    kp, vp = pool, -pool
    scr = ref.kv_pack(kp, vp, 1, 2, [4, 8])
    assert scr.shape == (1, 2, 2) + shape[2:]
    for j, p in enumerate([4, 8]):
        assert np.array_equal(scr[0, j, 0], kp[p, 1]) and np.array_equal(scr[0, j, 1], vp[p, 1])
    k2, v2 = np.zeros_like(kp), np.zeros_like(vp)
    ref.kv_scatter(k2, v2, 1, 2, [10, 3], scr)
    assert np.array_equal(k2[10, 1], kp[4, 1]) and np.array_equal(v2[3, 1], vp[8, 1])
    assert not k2[:, 0].any()


def _run_lifecycle(kv_rule, prompt_len, chunk, steps, use_tc, page_size=16, real_stage=False):
    """Positions appended over a request's life with kv_len from kv_rule;
    asserts every append stays inside the pages the table holds."""
    req = Request(prompt_len, chunk)
    positions = []
    for _ in range(steps):
        first, ql, flag, ctx, pages = req.step_args(use_tc, page_size)
        kv = int(kv_rule([first], [ql], [flag], use_tc, [ctx] if real_stage else None,
                         [pages], page_size)[0])
        assert kv <= pages * page_size, (first, ql, kv, pages)
        positions.extend(range(kv - ql, kv))
        req.finish_step()
    return positions


def _lifecycle_without_stages(kv_rule, prompt_len, chunk, steps, page_size):
    """--use-tensor-cores without the rows' real stages: at every step the
    rule either raises ValueError or gives the kv_len the real stage gives.
    Returns the number of steps that raised."""
    req = Request(prompt_len, chunk)
    raised = 0
    for _ in range(steps):
        first, ql, flag, ctx, pages = req.step_args(True, page_size)
        want = int(ref.kv_lens_for_step([first], [ql], [flag], True, [ctx])[0])
        try:
            got = int(kv_rule([first], [ql], [flag], True, None, [pages], page_size)[0])
        except ValueError:
            raised += 1
        else:
            assert got == want, (prompt_len, chunk, first, ql, pages)
        req.finish_step()
    return raised


def test_kv_len_rule_against_request_lifecycle():
    pos = _run_lifecycle(ref.kv_lens_for_step, 37, 16, 8, False)
    # Every token position is appended exactly once, in order.
    assert pos == list(range(len(pos)))
    pos = _run_lifecycle(ref.kv_lens_for_step, 37, 16, 8, True, real_stage=True)
    assert pos == list(range(len(pos)))


def test_kv_len_rule_with_tensor_cores_over_random_lifecycles():
    """--use-tensor-cores flags every row as prefill (request.py:667-670):
    given the rows' real stages, every position is appended exactly once and
    inside the blocks the table holds over random prompts and chunk sizes,
    one-token tail chunks included; without them the rule never returns a
    wrong kv_len, it raises. Oracle and library alike."""
    from kunserve_amd import kv_lens_for_step as lib_rule

    rng = np.random.default_rng(11)
    tails = 0
    for _ in range(300):
        chunk = int(rng.integers(2, 80))
        prompt = int(rng.integers(1, 400))
        tails += prompt > 1 and prompt % chunk == 1
        for rule in (ref.kv_lens_for_step, lib_rule):
            for ps in (4, 16):
                pos = _run_lifecycle(rule, prompt, chunk, 12, True, ps, real_stage=True)
                assert pos == list(range(len(pos)))
                _lifecycle_without_stages(rule, prompt, chunk, 12, ps)
    assert tails > 0


def test_tensor_cores_without_stages_raises_on_ambiguous_rows():
    """A prompt one token longer than a chunk multiple ends in a one-token
    chunk at first index > 0, which the all-prefill flags cannot tell from a
    decode row; given the rows' real stages the rule appends every position
    once; without them it raises at that chunk (and at decode rows whose
    table could hold their position), rather than writing K/V one position
    off. A decode row whose table is too short for position `first` is
    settled by its page count, and a one-token prompt (first index 0) needs
    no help."""
    from kunserve_amd import kv_lens_for_step as lib_rule

    for rule in (ref.kv_lens_for_step, lib_rule):
        pos = _run_lifecycle(rule, 33, 16, 6, True, real_stage=True)
        assert pos == list(range(36))
        assert _run_lifecycle(rule, 1, 16, 1, True) == [0]
        with pytest.raises(ValueError, match="is_context_stage|ambiguous"):
            _run_lifecycle(rule, 33, 16, 6, True)
        # the tail chunk (first 32, 3 pages of 16) and the decode row at
        # first 33 (3 pages) raise; the decode row at 48 (3 pages) does not
        assert rule([48], [1], [1], True, None, [3], 16).tolist() == [48]
        for first, pages in ((32, 3), (33, 3), (47, 3), (48, 4)):
            with pytest.raises(ValueError):
                rule([first], [1], [1], True, None, [pages], 16)
        # the tail row itself, without page counts
        with pytest.raises(ValueError):
            rule([32], [1], [1], True)
        assert _lifecycle_without_stages(rule, 513, 512, 4, 16) == 3   # all but the first chunk


def test_fused_page_ids():
    # P = 4 base pages, 3 instances: page 1 -> {1, 5, 9}; extend ids follow 12.
    assert ref.fused_page_ids(1, 4, 3) == [1, 5, 9]
    assert ref.extend_page_ids(12, 3) == [12, 13, 14]
    # instance rank 2 keeps fused id 8 + b
    assert ref.kept_page_id(3, 12, 3, 2) == 11
    # the kept id is one of the fused ids of that page
    assert ref.kept_page_id(3, 12, 3, 2) in ref.fused_page_ids(3, 4, 3)


@pytest.mark.parametrize("P,N,L,X", [(4, 2, 4, 3), (5, 4, 8, 2), (3, 1, 2, 1), (7, 8, 8, 0)])
def test_fused_slab_map_invariants(P, N, L, X):
    """The fused address map of the oracle, pinned by what the reference's
    block manager relies on:
    * a stale request of rank r keeps fused id r*P + b and its KV is not
      moved (kunserve/block_manager.py:755-760): local layer j of that id is
      model layer r*G + j of page b;
    * the fused ids convert_to_pipeline_format makes of free page b
      (:250-253) cover exactly the L layers of page b, and no other page;
    * extend ids (:262-269) address only the pages behind the base ones;
    * every slab of the pool is used by exactly one (fused id, local layer)."""
    G = L // N
    seen = {}
    for f in range((P + X) * N):
        for j in range(G):
            slab = ref.fused_slab(f, j, P, N, L)
            assert slab not in seen, f"slab {slab} used by {seen[slab]} and {(f, j)}"
            seen[slab] = (f, j)
    assert set(seen) == {(b, layer) for b in range(P + X) for layer in range(L)}
    for b in range(P):
        for r in range(N):
            kept = ref.kept_page_id(b, P * N, N, r)
            assert [ref.fused_slab(kept, j, P, N, L) for j in range(G)] == \
                [(b, r * G + j) for j in range(G)]
        slabs = {ref.fused_slab(f, j, P, N, L) for f in ref.fused_page_ids(b, P, N)
                 for j in range(G)}
        assert slabs == {(b, layer) for layer in range(L)}
    for f in ref.extend_page_ids(P * N, X * N):
        assert all(ref.fused_slab(f, j, P, N, L)[0] >= P for j in range(G))


def test_fused_pool_copy_is_an_element_loop_of_the_map():
    rng = np.random.default_rng(7)
    P, N, L, X = 3, 2, 4, 2
    pool = rng.permutation((P + X) * L * 2 * 4 * 8).reshape(P + X, L, 2, 4, 8)
    fused = ref.fused_pool_copy(pool, P, N)
    assert fused.shape == ((P + X) * N, L // N, 2, 4, 8)
    for f in range((P + X) * N):
        for j in range(L // N):
            page, layer = ref.fused_slab(f, j, P, N, L)
            for h in range(2):
                for t in range(4):
                    assert np.array_equal(fused[f, j, h, t], pool[page, layer, h, t])


# ------------------------------------------------------------------ rope

def _hf_rotate_half(x, pos, inv_freq):
    """The Hugging Face Llama form: x * cos + rotate_half(x) * sin with
    cos/sin of cat(freqs, freqs) (an independent formulation)."""
    freqs = np.outer(np.asarray(pos, np.float32), inv_freq).astype(np.float32)
    emb = np.concatenate([freqs, freqs], axis=-1).astype(np.float64)
    cos, sin = np.cos(emb)[:, None, :], np.sin(emb)[:, None, :]
    d = x.shape[-1]
    rot = np.concatenate([-x[..., d // 2:], x[..., : d // 2]], axis=-1)
    return x * cos + rot * sin


def _complex_interleaved(x, pos, inv_freq):
    """The original Llama form: consecutive pairs as complex numbers times
    e^(i * angle)."""
    ang = np.outer(np.asarray(pos, np.float32), inv_freq).astype(np.float32).astype(np.float64)
    z = x[..., 0::2] + 1j * x[..., 1::2]
    z = z * np.exp(1j * ang)[:, None, :]
    out = np.empty_like(x)
    out[..., 0::2], out[..., 1::2] = z.real, z.imag
    return out


@pytest.mark.parametrize("d", [64, 128])
def test_rope_matches_both_published_forms(d):
    rng = np.random.default_rng(d)
    x = rng.standard_normal((9, 3, d))
    pos = np.array([0, 1, 2, 17, 100, 511, 4095, 30000, 131071])
    inv = (1.0 / (np.float32(10000.0) ** (np.arange(0, d, 2, dtype=np.float32) / d))).astype(np.float32)
    np.testing.assert_allclose(ref.rope(x, pos, inv, False), _hf_rotate_half(x, pos, inv),
                               rtol=0, atol=1e-12)
    np.testing.assert_allclose(ref.rope(x, pos, inv, True), _complex_interleaved(x, pos, inv),
                               rtol=0, atol=1e-12)


def test_rope_closed_forms():
    rng = np.random.default_rng(3)
    d = 128
    x = rng.standard_normal((5, 2, d))
    inv = (2.0 ** -np.arange(d // 2, dtype=np.float64) / 4).astype(np.float32)  # exact fp32 angles
    for il in (False, True):
        # position 0 is the identity
        np.testing.assert_array_equal(ref.rope(x, np.zeros(5, np.int64), inv, il), x)
        # each pair keeps its norm
        y = ref.rope(x, np.arange(5) * 37, inv, il)
        pa = (x[..., 0::2], x[..., 1::2]) if il else (x[..., : d // 2], x[..., d // 2:])
        pb = (y[..., 0::2], y[..., 1::2]) if il else (y[..., : d // 2], y[..., d // 2:])
        np.testing.assert_allclose(pa[0] ** 2 + pa[1] ** 2, pb[0] ** 2 + pb[1] ** 2, atol=1e-12)
        # scores depend on the position difference only
        q, k = x[:1], x[1:2]
        s1 = np.sum(ref.rope(q, np.array([900]), inv, il) * ref.rope(k, np.array([700]), inv, il))
        s2 = np.sum(ref.rope(q, np.array([200]), inv, il) * ref.rope(k, np.array([0]), inv, il))
        assert abs(s1 - s2) < 1e-9
    # interleaved = half-split on de-interleaved dims
    perm = np.concatenate([np.arange(0, d, 2), np.arange(1, d, 2)])
    yh = ref.rope(x[..., perm], np.arange(5) * 11, inv, False)
    yi = ref.rope(x, np.arange(5) * 11, inv, True)
    np.testing.assert_allclose(yi[..., perm], yh, atol=1e-12)


def test_rope_append_positions_and_pages():
    rng = np.random.default_rng(4)
    ps, npg, hkv, hq, d = 16, 24, 2, 4, 64
    q_lens = np.array([3, 1, 20])
    kv = np.array([3, 40, 25], dtype=np.int64)   # prefixes 0, 39, 5
    need = (kv + ps - 1) // ps
    indptr = np.concatenate([[0], np.cumsum(need)])
    indices = rng.permutation(npg)[: indptr[-1]]
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)])
    T = int(q_indptr[-1])
    pos = ref.token_positions(kv, q_indptr)
    assert pos.tolist() == [0, 1, 2, 39] + list(range(5, 25))
    q = rng.standard_normal((T, hq, d)).astype(np.float16)
    kn = rng.standard_normal((T, hkv, d)).astype(np.float16)
    vn = rng.standard_normal((T, hkv, d)).astype(np.float16)
    k_pool = np.zeros((npg, 1, hkv, ps, d), np.float16)
    v_pool = np.zeros_like(k_pool)
    inv = (1.0 / (np.float32(10000.0) ** (np.arange(0, d, 2, dtype=np.float32) / d))).astype(np.float32)
    qr = ref.rope_append_kv(k_pool, v_pool, 0, indptr, indices, kv, q_indptr, q, kn, vn, inv, False)
    np.testing.assert_array_equal(qr, ref.rope(q, pos, inv, False).astype(np.float16))
    kr = ref.rope(kn, pos, inv, False).astype(np.float16)
    for t in range(T):
        b = int(np.searchsorted(q_indptr, t, side="right") - 1)
        page = indices[indptr[b] + pos[t] // ps]
        np.testing.assert_array_equal(k_pool[page, 0, :, pos[t] % ps], kr[t])
        np.testing.assert_array_equal(v_pool[page, 0, :, pos[t] % ps], vn[t])


def test_torch_cpu_restatement_matches_the_oracle():
    """The PyTorch-CPU decode that bench.py times as its CPU baseline computes
    the oracle's decode (fp32 vs float64: within 1e-5 on fp16 pages)."""
    from oracle import torch_cpu

    rng = np.random.default_rng(17)
    npg, L, hkv, ps, d = 40, 2, 4, 16, 64
    for hq in (4, 16):
        k = rng.standard_normal((npg, L, hkv, ps, d)).astype(np.float16)
        v = rng.standard_normal((npg, L, hkv, ps, d)).astype(np.float16)
        kv = np.array([0, 1, 17, 200, 96])
        need = (kv + ps - 1) // ps
        indptr = np.concatenate([[0], np.cumsum(need)])
        indices = rng.permutation(npg)[:indptr[-1]]
        q = rng.standard_normal((5, hq, d)).astype(np.float16)
        want = ref.decode_attention(q, k, v, 1, indptr, indices, kv, 0.125)
        got = torch_cpu.decode_attention(torch.from_numpy(q), torch.from_numpy(k),
                                         torch.from_numpy(v), 1, indptr, indices, kv, 0.125)
        np.testing.assert_allclose(got.numpy(), want, rtol=0, atol=1e-5)


def test_torch_prefill_restatement_matches_the_oracle():
    """The PyTorch prefill that the GPU tests run on the device as the
    full-size reference of the chunked-prefill workload, and that bench.py
    times as the prefill CPU baseline, computes the oracle's causal prefill
    (fp32 vs float64: within 1e-5 on fp16 pages), for MHA and GQA, ragged
    rows with and without prefixes, and a row subset."""
    from oracle import torch_cpu

    rng = np.random.default_rng(18)
    npg, L, hkv, ps, d = 60, 2, 2, 16, 64
    k = rng.standard_normal((npg, L, hkv, ps, d)).astype(np.float16)
    v = rng.standard_normal((npg, L, hkv, ps, d)).astype(np.float16)
    q_lens = np.array([1, 33, 7, 64])
    prefix = np.array([40, 0, 250, 100])
    kv = prefix + q_lens
    need = (kv + ps - 1) // ps
    indptr = np.concatenate([[0], np.cumsum(need)])
    indices = rng.permutation(npg)[:indptr[-1]]
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)])
    for hq in (2, 6):
        q = rng.standard_normal((int(q_lens.sum()), hq, d)).astype(np.float16)
        want = ref.prefill_attention(q, q_indptr, k, v, 1, indptr, indices, kv, 0.125)
        got = torch_cpu.prefill_attention(torch.from_numpy(q), q_indptr, torch.from_numpy(k),
                                          torch.from_numpy(v), 1, indptr, indices, kv, 0.125)
        np.testing.assert_allclose(got.numpy(), want, rtol=0, atol=1e-5)
        part = torch_cpu.prefill_attention(torch.from_numpy(q), q_indptr, torch.from_numpy(k),
                                           torch.from_numpy(v), 1, indptr, indices, kv, 0.125,
                                           rows=[2])
        np.testing.assert_array_equal(part.numpy()[q_indptr[2]:q_indptr[3]],
                                      got.numpy()[q_indptr[2]:q_indptr[3]])
        assert not part.numpy()[:q_indptr[2]].any() and not part.numpy()[q_indptr[3]:].any()


def test_torch_copy_restatement_matches_the_oracle():
    """The PyTorch block copy that bench.py times as the remap copy's CPU
    baseline moves the oracle's bytes."""
    from oracle import torch_cpu

    rng = np.random.default_rng(19)
    kp = rng.integers(-30000, 30000, (24, 3, 2, 4, 8)).astype(np.int16)
    vp = rng.integers(-30000, 30000, (24, 3, 2, 4, 8)).astype(np.int16)
    src, dst = rng.permutation(12)[:7], 12 + rng.permutation(12)[:7]
    kt, vt = torch.from_numpy(kp.copy()), torch.from_numpy(vp.copy())
    torch_cpu.copy_blocks(kt, vt, src, dst)
    ref.copy_blocks(kp, src, dst)
    ref.copy_blocks(vp, src, dst)
    assert np.array_equal(kt.numpy(), kp) and np.array_equal(vt.numpy(), vp)
