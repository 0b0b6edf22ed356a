"""Fused RoPE + K/V append prologue on the GPU vs the CPU oracle.

Rotated q and k agree with the oracle to one fp16 ulp plus 1e-6 (GPU
sincosf and rotation in fp32 against float64 cos/sin of the same fp32
angle); v and every pool entry the step does not own are bit-exact."""
import math

import numpy as np
import pytest
import torch

from kunserve_amd import AttentionStep, KVPool, rope_append_kv, rope_inv_freq
from oracle import paged_attention_ref as ref

from helpers import ATOL, compact_for_oracle, max_abs, random_pool, random_tensor, table_from_csr

pytestmark = pytest.mark.gpu


def make_rows(rng, q_lens, prefixes, ps, npg):
    kv = np.asarray(prefixes) + np.asarray(q_lens)
    need = (kv + ps - 1) // ps
    indptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
    indices = rng.permutation(npg)[:indptr[-1]].astype(np.int32)
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    return kv.astype(np.int32), indptr, indices, q_indptr


def within_one_ulp(got: np.ndarray, want: np.ndarray) -> bool:
    """One fp16 ulp of the rounded oracle value, with a 1e-6 floor: where
    x cos - y sin cancels to near zero the fp16 ulp is subnormal (6e-8), below
    the ~1e-7 absolute error of any fp32 evaluation."""
    want16 = want.astype(np.float16)
    tol = np.spacing(np.abs(want16)).astype(np.float64) + 1e-6
    return bool(np.all(np.abs(got.astype(np.float64) - want16.astype(np.float64)) <= tol))


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("interleave", [False, True])
@pytest.mark.parametrize("ps", [16, 64])
def test_rope_append_matches_oracle(device, d, interleave, ps):
    rng = np.random.default_rng(d + ps + interleave)
    hq, hkv = 8, 2
    q_lens, prefixes = [1, 5, 130, 1, 64], [0, 300, 17, 4000, 62]
    npg = 320 if ps == 16 else 120   # the rows need 290 and 74 pages
    kv, indptr, indices, q_indptr = make_rows(rng, q_lens, prefixes, ps, npg)
    pool = random_pool(npg, 2, hkv, ps, d, device, 1)
    k0, v0 = pool.k.cpu().numpy(), pool.v.cpu().numpy()
    T = int(q_indptr[-1])
    q = random_tensor((T, hq, d), device, 2)
    kn, vn = random_tensor((T, hkv, d), device, 3), random_tensor((T, hkv, d), device, 4)
    q_in = q.cpu().numpy()
    inv = rope_inv_freq(d, 10000.0, device)
    table = table_from_csr(indptr, indices, kv, device)
    rope_append_kv(pool, 1, table, torch.from_numpy(q_indptr).to(device), q, kn, vn, inv,
                   interleave)
    torch.cuda.synchronize()
    pos = ref.token_positions(kv, q_indptr)
    invn = inv.cpu().numpy()
    assert within_one_ulp(q.cpu().numpy(), ref.rope(q_in, pos, invn, interleave))
    want_k = ref.rope(kn.cpu().numpy(), pos, invn, interleave)
    k1, v1 = pool.k.cpu().numpy(), pool.v.cpu().numpy()
    # expected pools: the oracle append of (rotated k rounded, v) on the old pools
    ke, ve = k0.copy(), v0.copy()
    ref.append_kv(ke, ve, 1, indptr, indices, kv, q_indptr, want_k.astype(np.float16),
                  vn.cpu().numpy())
    assert np.array_equal(v1.view(np.int16), ve.view(np.int16))
    owned = np.zeros(k1.shape[:4], dtype=bool)
    for t, p in enumerate(pos):
        b = int(np.searchsorted(q_indptr, t, side="right") - 1)
        owned[indices[indptr[b] + p // ps], 1, :, p % ps] = True
    assert np.array_equal(k1[~owned].view(np.int16), k0[~owned].view(np.int16))
    assert within_one_ulp(k1[owned], ke[owned].astype(np.float64))


def test_attention_step_with_rope_matches_oracle(device):
    """pforward's attention stage with the fused prologue: rotate, append,
    attend (decode and chunked-prefill rows in one step)."""
    rng = np.random.default_rng(9)
    ps, npg, hq, hkv, d = 16, 200, 8, 2, 128
    pool = KVPool.allocate(npg, 2, hkv, ps, d, device)
    pool.k.copy_(random_pool(npg, 2, hkv, ps, d, device, 10).k)
    pool.v.copy_(random_pool(npg, 2, hkv, ps, d, device, 11).v)
    q_lens = np.array([1, 40, 1, 300])
    flags = np.array([0, 1, 0, 1])
    first = np.array([77, 60, 500, 0])          # decode: kv_len = first; prefill: first + q_len
    kv = np.where(flags == 0, first, first + q_lens)
    need = (kv + ps - 1) // ps
    perm = rng.permutation(npg)
    pages, o = [], 0
    for n in need:
        pages.append(perm[o:o + n].tolist())
        o += n
    step = AttentionStep(pool, hq, q_lens, first, flags, pages)
    T = int(q_lens.sum())
    q = random_tensor((T, hq, d), device, 12)
    k, v = random_tensor((T, hkv, d), device, 13), random_tensor((T, hkv, d), device, 14)
    q_in = q.cpu().numpy()
    k0, v0 = pool.k.cpu().numpy(), pool.v.cpu().numpy()
    inv = rope_inv_freq(d, 10000.0, device)
    out = step.run(1, q, k, v, rope=(inv, False))
    torch.cuda.synchronize()
    indptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
    indices = np.concatenate(pages).astype(np.int32)
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    q_rot = ref.rope_append_kv(k0, v0, 1, indptr, indices, kv, q_indptr, q_in, k.cpu().numpy(),
                               v.cpu().numpy(), inv.cpu().numpy(), False)
    want = ref.prefill_attention(q_rot, q_indptr, k0, v0, 1, indptr, indices, kv,
                                 1.0 / math.sqrt(d))
    assert max_abs(out, want) <= ATOL
