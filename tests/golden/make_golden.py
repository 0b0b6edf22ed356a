"""Writes the small golden vectors under tests/golden/ (inputs and expected
outputs, computed by the CPU oracle in float64).

The reference ships no golden vectors for this path (its native backend is
an empty submodule), so these fixtures freeze the oracle's answers on tiny,
seeded cases: tests/test_golden.py re-derives them on the CPU (oracle drift)
and tests/test_gpu_golden.py checks the HIP kernels against them.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import paged_attention_ref as ref  # noqa: E402


def tables(rng, kv_len, page_size, num_pages):
    need = (np.asarray(kv_len) + page_size - 1) // page_size
    indptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
    indices = rng.permutation(num_pages)[:indptr[-1]].astype(np.int32)
    return indptr, indices


def decode_case(seed=2001):
    rng = np.random.default_rng(seed)
    npg, L, hkv, ps, d, hq = 16, 2, 1, 16, 128, 4
    kv = np.array([1, 17, 64, 100, 0], dtype=np.int32)
    indptr, indices = tables(rng, kv, ps, npg)
    k = (rng.standard_normal((npg, L, hkv, ps, d)) / math.sqrt(d)).astype(np.float16)
    v = rng.standard_normal((npg, L, hkv, ps, d)).astype(np.float16)
    q = rng.standard_normal((len(kv), hq, d)).astype(np.float16)
    out = ref.decode_attention(q, k, v, 1, indptr, indices, kv, 1 / math.sqrt(d))
    return dict(k=k, v=v, q=q, indptr=indptr, indices=indices, kv_len=kv, layer=np.int32(1),
                out=out.astype(np.float32))


def prefill_case(seed=2002):
    rng = np.random.default_rng(seed)
    npg, L, hkv, ps, d, hq = 10, 1, 2, 16, 128, 4
    q_lens = np.array([3, 40, 1], dtype=np.int32)
    prefix = np.array([0, 40, 20], dtype=np.int32)
    kv = (q_lens + prefix).astype(np.int32)
    indptr, indices = tables(rng, kv, ps, npg)
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    k = rng.standard_normal((npg, L, hkv, ps, d)).astype(np.float16)
    v = rng.standard_normal((npg, L, hkv, ps, d)).astype(np.float16)
    q = (rng.standard_normal((int(q_indptr[-1]), hq, d)) / math.sqrt(d)).astype(np.float16)
    out = ref.prefill_attention(q, q_indptr, k, v, 0, indptr, indices, kv, 1 / math.sqrt(d))
    return dict(k=k, v=v, q=q, q_indptr=q_indptr, indptr=indptr, indices=indices, kv_len=kv,
                out=out.astype(np.float32))


def append_case(seed=2003):
    rng = np.random.default_rng(seed)
    npg, L, hkv, ps, d = 8, 2, 1, 16, 64
    q_lens = np.array([5, 1, 20], dtype=np.int32)
    prefix = np.array([14, 31, 0], dtype=np.int32)
    kv = (q_lens + prefix).astype(np.int32)
    indptr, indices = tables(rng, kv, ps, npg)
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    k = rng.standard_normal((npg, L, hkv, ps, d)).astype(np.float16)
    v = rng.standard_normal((npg, L, hkv, ps, d)).astype(np.float16)
    T = int(q_indptr[-1])
    k_new = rng.standard_normal((T, hkv, d)).astype(np.float16)
    v_new = rng.standard_normal((T, hkv, d)).astype(np.float16)
    k_out, v_out = k.copy(), v.copy()
    ref.append_kv(k_out, v_out, 1, indptr, indices, kv, q_indptr, k_new, v_new)
    return dict(k=k, v=v, k_new=k_new, v_new=v_new, q_indptr=q_indptr, indptr=indptr,
                indices=indices, kv_len=kv, layer=np.int32(1), k_out=k_out, v_out=v_out)


def copy_case(seed=2004):
    rng = np.random.default_rng(seed)
    shape = (10, 3, 1, 16, 64)
    k = rng.integers(-30000, 30000, shape).astype(np.int16)
    v = rng.integers(-30000, 30000, shape).astype(np.int16)
    ids = rng.permutation(10)
    src, dst = ids[:5].astype(np.int32), ids[5:10].astype(np.int32)
    k_out, v_out = k.copy(), v.copy()
    ref.copy_blocks(k_out, src, dst)
    ref.copy_blocks(v_out, src, dst)
    scratch = ref.kv_pack(k, v, 1, 3, src)
    return dict(k=k, v=v, src=src, dst=dst, k_out=k_out, v_out=v_out, pack_scratch=scratch)


CASES = {"decode": decode_case, "prefill": prefill_case, "append": append_case,
         "copy": copy_case}


def main():
    for name, make in CASES.items():
        path = HERE / f"{name}.npz"
        np.savez_compressed(path, **make())
        print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
