"""Randomised parity of decode and chunked prefill against the CPU oracle
over head layouts, head dims, page sizes, dtypes, partition lengths and
ragged or empty rows. hypothesis draws the cases from a fixed seed
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
       ps=st.sampled_from([4, 16, 64, 256]),
       rows=st.lists(st.tuples(st.integers(1, 200), st.integers(0, 800)), min_size=1,
                     max_size=4),
       bf16=st.booleans(), seed=st.integers(0, 2**16))
def test_prefill_random_cases(device, hkv, ratio, ps, rows, bf16, seed):
    dtype = torch.bfloat16 if bf16 else torch.float16
    rng = np.random.default_rng(seed)
    q_lens = np.array([r[0] for r in rows], dtype=np.int32)
    kv, indptr, indices, npg = _rows(rng, [q + p for q, p in rows], ps)
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    hq = hkv * ratio
    pool = random_pool(npg, 1, hkv, ps, 128, device, seed, dtype=dtype)
    q = random_tensor((int(q_indptr[-1]), hq, 128), device, seed + 1, dtype=dtype)
    plan = PrefillPlan(q_indptr, kv, hq, hkv, device)
    out = paged_prefill(pool, 0, table_from_csr(indptr, indices, kv, device),
                        torch.from_numpy(q_indptr).to(device), q, plan)
    torch.cuda.synchronize()
    k, v, ip, ix = compact_for_oracle(pool, 0, indptr, indices)
    want = ref.prefill_attention(to_numpy(q), q_indptr, k, v, 0, ip, ix, kv, 1 / math.sqrt(128))
    assert max_abs(out, want) <= (ATOL_BF16 if bf16 else ATOL)
