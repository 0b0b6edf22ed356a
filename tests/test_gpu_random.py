"""Randomised parity against the CPU oracle: decode and chunked prefill
(tolerance) over head layouts, head dims, page sizes, dtypes, partition
lengths and ragged or empty rows; block copy, pack, scatter and append
(bit-exact) over pool geometries, layer ranges and id lists. hypothesis draws the cases from a fixed seed
(derandomize), so every run checks the same ones; each is small enough
for the oracle to finish in well under a second."""
import math

import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings, strategies as st

from kunserve_amd import DecodePlan, PrefillPlan, paged_decode, paged_prefill
from oracle import paged_attention_ref as ref

from helpers import (ATOL, ATOL_BF16, compact_for_oracle, max_abs, random_pool, random_tensor,
                     table_from_csr, to_numpy)

pytestmark = pytest.mark.gpu

RANDOM = settings(max_examples=80, deadline=None, derandomize=True, database=None,
                  suppress_health_check=[HealthCheck.too_slow,
                                         HealthCheck.function_scoped_fixture])


def _rows(rng, kv, ps):
    kv = np.asarray(kv, dtype=np.int32)
    need = (kv + ps - 1) // ps
    indptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
    npg = int(indptr[-1]) + 3
    indices = rng.permutation(npg)[:indptr[-1]].astype(np.int32)
    return kv, indptr, indices, npg


@RANDOM
@given(hkv=st.sampled_from([1, 2, 4, 8]), ratio=st.sampled_from([1, 2, 3, 4, 8]),
       d=st.sampled_from([64, 128, 256]), ps=st.sampled_from([4, 8, 16, 32, 256]),
       kv=st.lists(st.integers(0, 3000), min_size=1, max_size=6),
       part=st.sampled_from([0, 256, 512]), bf16=st.booleans(), seed=st.integers(0, 2**16))
def test_decode_random_cases(device, hkv, ratio, d, ps, kv, part, bf16, seed):
    dtype = torch.bfloat16 if bf16 else torch.float16
    rng = np.random.default_rng(seed)
    kv[0] = max(kv[0], 1)
    kv, indptr, indices, npg = _rows(rng, kv, ps)
    hq = hkv * ratio
    pool = random_pool(npg, 1, hkv, ps, d, device, seed, dtype=dtype)
    q = random_tensor((len(kv), hq, d), device, seed + 1, dtype=dtype)
    plan = DecodePlan(kv, hq, hkv, device, part_tokens=part)
    out = paged_decode(pool, 0, table_from_csr(indptr, indices, kv, device), q, plan)
    torch.cuda.synchronize()
    k, v, ip, ix = compact_for_oracle(pool, 0, indptr, indices)
    want = ref.decode_attention(to_numpy(q), k, v, 0, ip, ix, kv, 1 / math.sqrt(d))
    assert max_abs(out, want) <= (ATOL_BF16 if bf16 else ATOL)
    assert torch.all(out[torch.from_numpy(kv == 0).to(device)] == 0)


@RANDOM
@given(hkv=st.sampled_from([1, 2, 4]), ratio=st.sampled_from([1, 2, 4]),
       d=st.sampled_from([64, 128, 256]), ps=st.sampled_from([4, 16, 64, 256]),
       rows=st.lists(st.tuples(st.integers(1, 200), st.integers(0, 800)), min_size=1,
                     max_size=4),
       bf16=st.booleans(), seed=st.integers(0, 2**16))
def test_prefill_random_cases(device, hkv, ratio, d, ps, rows, bf16, seed):
    _check_prefill(device, hkv, ratio, d, ps, rows, bf16, seed)


@settings(RANDOM, max_examples=40)
@given(hkv=st.sampled_from([1, 2, 4]), ratio=st.sampled_from([1, 2, 4]),
       d=st.sampled_from([64, 128, 256]), ps=st.sampled_from([4, 16, 64, 256]),
       rows=st.lists(st.tuples(st.integers(1, 1600), st.integers(0, 3000)), min_size=1,
                     max_size=3),
       bf16=st.booleans(), seed=st.integers(0, 2**16))
def test_prefill_random_long_rows(device, hkv, ratio, d, ps, rows, bf16, seed):
    """Rows of several q tiles, diagonal tiles deep into long prefixes, and
    steps small enough that the plan splits the KV range."""
    _check_prefill(device, hkv, ratio, d, ps, rows, bf16, seed)


def _check_prefill(device, hkv, ratio, d, ps, rows, bf16, seed):
    dtype = torch.bfloat16 if bf16 else torch.float16
    rng = np.random.default_rng(seed)
    q_lens = np.array([r[0] for r in rows], dtype=np.int32)
    kv, indptr, indices, npg = _rows(rng, [q + p for q, p in rows], ps)
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    hq = hkv * ratio
    pool = random_pool(npg, 1, hkv, ps, d, device, seed, dtype=dtype)
    q = random_tensor((int(q_indptr[-1]), hq, d), device, seed + 1, dtype=dtype)
    plan = PrefillPlan(q_indptr, kv, hq, hkv, device, head_dim=d)
    out = paged_prefill(pool, 0, table_from_csr(indptr, indices, kv, device),
                        torch.from_numpy(q_indptr).to(device), q, plan)
    torch.cuda.synchronize()
    k, v, ip, ix = compact_for_oracle(pool, 0, indptr, indices)
    want = ref.prefill_attention(to_numpy(q), q_indptr, k, v, 0, ip, ix, kv, 1 / math.sqrt(d))
    assert max_abs(out, want) <= (ATOL_BF16 if bf16 else ATOL)


BYTES = settings(max_examples=25, deadline=None, derandomize=True, database=None,
                 suppress_health_check=[HealthCheck.too_slow,
                                        HealthCheck.function_scoped_fixture])


def _bits_pool(npg, layers, hkv, ps, d, device, seed, dtype):
    """K and V pools of random 16-bit patterns (bit-exact checks only)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    shape = (npg, layers, hkv, ps, d)
    mk = lambda: torch.randint(-32768, 32767, shape, generator=g, device=device,
                               dtype=torch.int16).view(dtype)
    from kunserve_amd import KVPool
    return KVPool(mk(), mk())


def _bits(t):
    return t.view(torch.int16).cpu().numpy()


@BYTES
@given(layers=st.integers(1, 4), hkv=st.sampled_from([1, 2, 8]),
       ps=st.sampled_from([4, 16, 256]), d=st.sampled_from([64, 128, 256]),
       n=st.integers(1, 24), bf16=st.booleans(), seed=st.integers(0, 2**16))
def test_copy_pack_scatter_random_cases(device, layers, hkv, ps, d, n, bf16, seed):
    from kunserve_amd import copy_blocks, kv_pack, kv_scatter
    dtype = torch.bfloat16 if bf16 else torch.float16
    rng = np.random.default_rng(seed)
    npg = 2 * n + 5
    pool = _bits_pool(npg, layers, hkv, ps, d, device, seed, dtype)
    k0, v0 = _bits(pool.k), _bits(pool.v)
    perm = rng.permutation(npg)
    src, dst = perm[:n].tolist(), perm[n:2 * n].tolist()
    copy_blocks(pool, src, dst)
    torch.cuda.synchronize()
    ref.copy_blocks(k0, src, dst)
    ref.copy_blocks(v0, src, dst)
    assert np.array_equal(_bits(pool.k), k0) and np.array_equal(_bits(pool.v), v0)

    lb = int(rng.integers(0, layers))
    le = int(rng.integers(lb + 1, layers + 1))
    ids = rng.integers(0, npg, n).tolist()          # repeats allowed when gathering
    scratch = kv_pack(pool, lb, le, ids)
    torch.cuda.synchronize()
    want = ref.kv_pack(k0, v0, lb, le, ids)
    assert np.array_equal(_bits(scratch)[:want.size].reshape(want.shape), want)

    dst_ids = rng.permutation(npg)[:n].tolist()     # distinct when scattering
    incoming = torch.randint(-32768, 32767, (want.size,), device=device,
                             dtype=torch.int16).view(dtype)
    kv_scatter(pool, lb, le, dst_ids, incoming)
    torch.cuda.synchronize()
    ref.kv_scatter(k0, v0, lb, le, dst_ids, _bits(incoming).reshape(want.shape))
    assert np.array_equal(_bits(pool.k), k0) and np.array_equal(_bits(pool.v), v0)


@BYTES
@given(layers=st.integers(1, 3), hkv=st.sampled_from([1, 2, 8]),
       ps=st.sampled_from([4, 16, 256]), d=st.sampled_from([64, 128, 256]),
       rows=st.lists(st.tuples(st.integers(1, 80), st.integers(0, 600)), min_size=1,
                     max_size=5),
       bf16=st.booleans(), seed=st.integers(0, 2**16))
def test_append_random_cases(device, layers, hkv, ps, d, rows, bf16, seed):
    from kunserve_amd import append_kv
    dtype = torch.bfloat16 if bf16 else torch.float16
    rng = np.random.default_rng(seed)
    q_lens = np.array([r[0] for r in rows], dtype=np.int32)
    kv, indptr, indices, npg = _rows(rng, [q + p for q, p in rows], ps)
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    pool = _bits_pool(npg, layers, hkv, ps, d, device, seed, dtype)
    k0, v0 = _bits(pool.k), _bits(pool.v)
    T = int(q_indptr[-1])
    kn = torch.randint(-32768, 32767, (T, hkv, d), device=device, dtype=torch.int16).view(dtype)
    vn = torch.randint(-32768, 32767, (T, hkv, d), device=device, dtype=torch.int16).view(dtype)
    layer = int(rng.integers(0, layers))
    append_kv(pool, layer, table_from_csr(indptr, indices, kv, device),
              torch.from_numpy(q_indptr).to(device), kn, vn)
    torch.cuda.synchronize()
    ref.append_kv(k0, v0, layer, indptr, indices, kv, q_indptr, _bits(kn), _bits(vn))
    assert np.array_equal(_bits(pool.k), k0) and np.array_equal(_bits(pool.v), v0)
