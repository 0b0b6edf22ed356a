"""The C ABI library loads and exports exactly what include/kunserve_hip.h
declares; host-only entry points behave (no GPU needed)."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from kunserve_amd import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "kunserve_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kunserve_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    names = declared_functions()
    assert len(names) >= 14
    lib = _lib.lib()
    for name in names:
        assert hasattr(lib, name), f"{name} declared in the header but not exported"
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"


def test_version_and_error_channel():
    lib = _lib.lib()
    assert lib.kunserve_version() == 300
    assert lib.kunserve_last_error() == b""


def test_decode_plan_covers_every_token_once():
    rng = np.random.default_rng(0)
    kv = rng.integers(0, 5000, 37).astype(np.int32)
    kv[3] = 0
    for hq, hkv in [(32, 32), (32, 8), (64, 8), (12, 4)]:
        cap = _lib.lib().kunserve_decode_plan_bound(kv.ctypes.data, kv.size)
        buf = np.zeros(cap, dtype=np.int32)
        info = _lib.DecodePlanInfo()
        _lib.call("kunserve_decode_plan", kv.ctypes.data, kv.size, hq, hkv, 256, 0,
                  buf.ctypes.data, cap, ctypes.byref(info))
        work = _check_lanes(buf[:4 * info.num_work].reshape(-1, 4))
        merges = buf[4 * info.num_work:info.plan_ints].reshape(-1, 4)
        assert info.group_size in (1, 2, 4, 8) and (hq // hkv) % info.group_size == 0
        covered = np.zeros(kv.size, dtype=np.int64)
        for seq, b, e, slot in work:
            assert 0 <= b <= e <= kv[seq] and e - b <= info.part_tokens
            covered[seq] += e - b
        assert np.array_equal(covered, kv)
        slots = sorted(work[work[:, 3] >= 0, 3].tolist())
        assert slots == list(range(info.num_slots))
        for seq, s0, n, _ in merges:
            assert n > 1 and set(work[work[:, 0] == seq, 3]) == set(range(s0, s0 + n))
        single = [s for s in range(kv.size) if s not in set(merges[:, 0])]
        assert all((work[work[:, 0] == s, 3] == -1).all() for s in single)


def _check_lanes(records):
    """The decode plan's records are 8 XCD lanes interleaved (record 8 r + x
    is entry r of lane x): each lane's items come longest first, then only
    padding (seq -1). Returns the items."""
    assert records.shape[0] % 8 == 0
    for x in range(8):
        lane = records[x::8]
        real = lane[:, 0] >= 0
        n = int(real.sum())
        assert real[:n].all() and not real[n:].any(), "padding only at a lane's end"
        lengths = lane[:n, 2] - lane[:n, 1]
        assert np.all(np.diff(lengths) <= 0), "a lane is ordered longest first"
    return records[records[:, 0] >= 0]


def test_decode_plan_weights_odd_xcds():
    """Lanes are dealt longest first to the XCD that would finish the item
    first, the odd XCDs at 0.93 of the even ones' rate: with equal items the
    odd lanes get fewer, and the weighted loads end within one item."""
    kv = np.full(512, 512, dtype=np.int32)
    cap = _lib.lib().kunserve_decode_plan_bound(kv.ctypes.data, kv.size)
    buf = np.zeros(cap, dtype=np.int32)
    info = _lib.DecodePlanInfo()
    _lib.call("kunserve_decode_plan", kv.ctypes.data, kv.size, 32, 32, 256, 512,
              buf.ctypes.data, cap, ctypes.byref(info))
    rec = buf[:4 * info.num_work].reshape(-1, 4)
    counts = [int((rec[x::8, 0] >= 0).sum()) for x in range(8)]
    assert sum(counts) == 512
    assert min(counts[0::2]) > max(counts[1::2]), counts
    finish = [counts[x] * (512 + 32) / (1.0 if x % 2 == 0 else 0.93) for x in range(8)]
    assert max(finish) - min(finish) <= (512 + 32) / 0.93


def _auto_decode_plan(kv, hq, hkv, num_cus=256):
    kv = np.asarray(kv, dtype=np.int32)
    cap = _lib.lib().kunserve_decode_plan_bound(kv.ctypes.data, kv.size)
    buf = np.zeros(cap, dtype=np.int32)
    info = _lib.DecodePlanInfo()
    _lib.call("kunserve_decode_plan", kv.ctypes.data, kv.size, hq, hkv, num_cus, 0,
              buf.ctypes.data, cap, ctypes.byref(info))
    return info


def test_decode_plan_keeps_whole_rows_in_short_launches():
    """The automatic partition keeps whole rows (no merge pass) when the
    launch is short, whole rows already give every CU an item and no row
    is longer than two minimum partitions; longer launches keep their
    splits."""
    from kunserve_amd import workloads
    w = workloads.single_layer_decode()       # 8 rows x 32 heads, contexts U[128, 512]
    info = _auto_decode_plan(w.kv_len, 32, 32)
    assert info.num_merge == 0 and info.num_work == 8 and info.part_tokens == 512
    # fewer row-head items than CUs: rows stay split for parallelism
    info = _auto_decode_plan(w.kv_len, 32, 32, num_cus=1024)
    assert info.part_tokens == 256 and info.num_merge > 0
    # a row longer than two minimum partitions: split
    info = _auto_decode_plan(np.r_[w.kv_len, 600], 32, 32)
    assert info.part_tokens == 256 and info.num_merge > 0
    # the Llama-2-7B, Llama-3-8B GQA and Llama-2-70B workloads take the
    # longest partitions: 7B rows are then whole (no merge launch)
    w = workloads.llama2_7b_decode()
    info = _auto_decode_plan(w.kv_len, 32, 32)
    assert info.part_tokens == 4096 and info.num_merge == 0
    w = workloads.llama3_8b_gqa_decode()
    assert _auto_decode_plan(w.kv_len, 32, 8).part_tokens == 4096
    w = workloads.kv_remap().decode
    assert _auto_decode_plan(w.kv_len, 64, 8).part_tokens == 4096


def test_decode_plan_automatic_partition_bounds():
    """The automatic partition keeps the longest item within 3/4 of a CU's
    share of the launch and gives every CU at least 4 workgroups: one row
    of 32768 tokens over 32 heads (a CU's share 4096 tokens) is cut into
    1024-token partitions (1024 workgroups on 256 CUs), and 16 rows of
    4096 tokens over 32 heads into 2048-token ones (1024 workgroups)."""
    info = _auto_decode_plan(np.array([32768], dtype=np.int32), 32, 32)
    assert info.part_tokens == 1024 and info.num_merge == 1
    info = _auto_decode_plan(np.full(16, 4096, dtype=np.int32), 32, 32)
    assert info.part_tokens == 2048


def test_decode_plan_rejects_bad_arguments():
    kv = np.array([10, 20], dtype=np.int32)
    buf = np.zeros(64, dtype=np.int32)
    info = _lib.DecodePlanInfo()
    with pytest.raises(_lib.KunserveError, match="multiple"):
        _lib.call("kunserve_decode_plan", kv.ctypes.data, 2, 30, 8, 256, 0, buf.ctypes.data,
                  64, ctypes.byref(info))
    with pytest.raises(_lib.KunserveError, match="part_tokens"):
        _lib.call("kunserve_decode_plan", kv.ctypes.data, 2, 8, 8, 256, 100, buf.ctypes.data,
                  64, ctypes.byref(info))
    with pytest.raises(_lib.KunserveError) as e:
        _lib.call("kunserve_decode_plan", kv.ctypes.data, 2, 8, 8, 256, 0, buf.ctypes.data, 2,
                  ctypes.byref(info))
    assert e.value.code == _lib.ENOSPC


def _prefill_plan(q_indptr, kv, hq, hkv, num_cus=256, head_dim=128):
    cap = _lib.lib().kunserve_prefill_plan_bound(q_indptr.ctypes.data, len(kv), hq, head_dim)
    buf = np.full(cap, -7, dtype=np.int32)
    info = _lib.PrefillPlanInfo()
    _lib.call("kunserve_prefill_plan", q_indptr.ctypes.data, kv.ctypes.data, len(kv), hq, hkv,
              head_dim, num_cus, buf.ctypes.data, cap, ctypes.byref(info))
    assert info.head_dim == head_dim
    items = buf[:6 * info.num_tiles].reshape(-1, 6)
    merges = buf[6 * info.num_tiles:info.plan_ints].reshape(-1, 5)
    return info, items, merges


def _check_prefill_plan(q_indptr, q_lens, kv, hq, hkv, info, items, merges):
    """Every (row, q tile, q head) covers its visible KV range [0, tile end)
    exactly once, split ranges are tile-aligned and contiguous, slots are
    distinct, and each split item has one merge record."""
    tq = info.tile_q
    n = len(kv)
    assert info.num_tiles % 8 == 0 and info.num_tiles == len(items)
    assert np.all(items[items[:, 0] < 0][:, 5] == -1)
    real = items[items[:, 0] >= 0]
    ranges = {}
    for b, q0, h, lo, hi, slot in real.tolist():
        ranges.setdefault((b, q0, h), []).append((lo, hi, slot))
    want = {(b, q0, h) for b in range(n) for q0 in range(0, int(q_lens[b]), tq)
            for h in range(hq)}
    assert set(ranges) == want
    slots = []
    merged = {(b, q0, h): (s0, cnt) for b, q0, h, s0, cnt in merges.tolist()}
    assert len(merged) == len(merges) == info.num_merge
    for (b, q0, h), rs in ranges.items():
        end = int(kv[b]) - int(q_lens[b]) + min(q0 + tq, int(q_lens[b]))
        rs.sort()
        assert rs[0][0] == 0 and rs[-1][1] == end
        for (lo1, hi1, _), (lo2, _, _) in zip(rs, rs[1:]):
            assert hi1 == lo2 and hi1 % 64 == 0
        if len(rs) == 1:
            assert rs[0][2] == -1 and (b, q0, h) not in merged
        else:
            s0, cnt = merged[(b, q0, h)]
            assert cnt == len(rs) and [r[2] for r in rs] == list(range(s0, s0 + cnt))
            assert all(hi - lo >= 64 * 4 or hi == end for lo, hi, _ in rs)
            slots += [r[2] for r in rs]
    assert sorted(slots) == list(range(info.num_slots))
    ws = _lib.lib().kunserve_prefill_workspace_bytes(ctypes.byref(info))
    assert ws == info.num_slots * tq * (info.head_dim + 2) * 4


@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("hq,hkv,n", [(4, 4, 3), (8, 2, 3), (32, 32, 16), (1, 1, 1)])
def test_prefill_plan_covers_every_tile_once(hq, hkv, n, head_dim):
    rng = np.random.default_rng(hq + n)
    q_lens = rng.integers(0, 900, n)
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    kv = (q_lens + rng.integers(0, 3000, n)).astype(np.int32)
    info, items, merges = _prefill_plan(q_indptr, kv, hq, hkv, head_dim=head_dim)
    assert info.tile_q == (128 if head_dim == 256 else 256)
    _check_prefill_plan(q_indptr, q_lens, kv, hq, hkv, info, items, merges)
    # items that read the same K/V (row, KV head) sit on one XCD
    xcd = {}
    for L, (b, q0, h, lo, hi, slot) in enumerate(items.tolist()):
        if b >= 0:
            xcd.setdefault((b, h // (hq // hkv)), set()).add(L % 8)
    if len(xcd) >= 16:
        assert all(len(v) == 1 for v in xcd.values())


@pytest.mark.parametrize("num_cus", [0, 64, 256, 1024])
def test_prefill_plan_splits_small_steps(num_cus):
    """A step with fewer q-tile items than CUs (one long row: the last step
    of a chunked prefill, 32 heads x 512 / tile_q items) is split over about
    one workgroup per CU; a step with enough items is not."""
    q_lens = np.array([512], dtype=np.int64)
    kv = np.array([4806], dtype=np.int32)
    q_indptr = np.array([0, 512], dtype=np.int32)
    info, items, merges = _prefill_plan(q_indptr, kv, 32, 32, num_cus)
    _check_prefill_plan(q_indptr, q_lens, kv, 32, 32, info, items, merges)
    cus = num_cus or 256
    n_items = -(-512 // info.tile_q) * 32
    real = int((items[:, 0] >= 0).sum())
    if cus <= n_items:
        assert info.num_merge == 0 and real == n_items
    else:
        assert info.num_merge == n_items and info.kv_chunk % 64 == 0 and info.kv_chunk >= 256
        assert 0.75 * cus <= real <= cus + n_items
    big = np.full(16, 512, dtype=np.int64)
    qi = np.concatenate([[0], np.cumsum(big)]).astype(np.int32)
    kvb = np.full(16, 2048, dtype=np.int32)
    info, items, merges = _prefill_plan(qi, kvb, 32, 32, 256)
    assert info.num_merge == 0 and info.num_slots == 0 and info.kv_chunk == 0


def test_prefill_plan_rejects_short_kv():
    q_indptr = np.array([0, 300, 301, 301 + 512], dtype=np.int32)
    bad = np.array([5, 1, 512], dtype=np.int32)   # kv_len shorter than q_len
    buf = np.zeros(64, dtype=np.int32)
    info = _lib.PrefillPlanInfo()
    with pytest.raises(_lib.KunserveError):
        _lib.call("kunserve_prefill_plan", q_indptr.ctypes.data, bad.ctypes.data, 3, 4, 4, 128,
                  0, buf.ctypes.data, 64, ctypes.byref(info))


@pytest.mark.parametrize("head_dim", [32, 96, 512])
def test_prefill_plan_rejects_unsupported_head_dims(head_dim):
    q_indptr = np.array([0, 8], dtype=np.int32)
    kv = np.array([8], dtype=np.int32)
    assert _lib.lib().kunserve_prefill_plan_bound(q_indptr.ctypes.data, 1, 4, head_dim) == -1
    buf = np.zeros(64, dtype=np.int32)
    info = _lib.PrefillPlanInfo()
    with pytest.raises(_lib.KunserveError) as e:
        _lib.call("kunserve_prefill_plan", q_indptr.ctypes.data, kv.ctypes.data, 1, 4, 4,
                  head_dim, 0, buf.ctypes.data, 64, ctypes.byref(info))
    assert e.value.code == _lib.EUNSUPPORTED


def test_swap_rejects_out_of_range_ids_before_any_copy():
    src = np.array([0, 9], dtype=np.int64)
    dst = np.array([1, 2], dtype=np.int64)
    dummy = ctypes.c_void_p(16)   # never dereferenced: validation fails first
    with pytest.raises(_lib.KunserveError) as e:
        _lib.call("kunserve_swap_blocks", src.ctypes.data, dst.ctypes.data, 2, 0, dummy, dummy,
                  4, dummy, dummy, 8, 1024, None)
    assert e.value.code == _lib.ERANGE


# ------------------------------------------------------------------------
# Randomised plan properties (hypothesis): the coverage invariants above on
# arbitrary batches, head layouts, CU counts and partition sizes.

from hypothesis import HealthCheck, given, settings, strategies as st  # noqa: E402

HEADS = [(1, 1), (4, 4), (8, 2), (12, 4), (32, 8), (64, 8), (32, 32), (6, 2)]


@settings(max_examples=60, deadline=None, suppress_health_check=[HealthCheck.too_slow])
@given(kv=st.lists(st.integers(0, 20000), min_size=0, max_size=24),
       heads=st.sampled_from(HEADS),
       num_cus=st.sampled_from([0, 1, 64, 256, 1024]),
       part=st.sampled_from([0, 256, 320, 512, 1024, 4096]))
def test_decode_plan_properties(kv, heads, num_cus, part):
    hq, hkv = heads
    kv = np.asarray(kv, dtype=np.int32)
    cap = _lib.lib().kunserve_decode_plan_bound(kv.ctypes.data if kv.size else None, kv.size)
    buf = np.zeros(max(cap, 1), dtype=np.int32)
    info = _lib.DecodePlanInfo()
    _lib.call("kunserve_decode_plan", kv.ctypes.data if kv.size else None, kv.size, hq, hkv,
              num_cus, part, buf.ctypes.data, cap, ctypes.byref(info))
    work = _check_lanes(buf[:4 * info.num_work].reshape(-1, 4))
    merges = buf[4 * info.num_work:info.plan_ints].reshape(-1, 4)
    assert part == 0 or info.part_tokens == part
    covered = np.zeros(kv.size, dtype=np.int64)
    for seq, b, e, slot in work:
        assert 0 <= b <= e <= kv[seq] and e - b <= info.part_tokens
        covered[seq] += e - b
    assert np.array_equal(covered, kv)
    assert sorted(work[work[:, 3] >= 0, 3].tolist()) == list(range(info.num_slots))
    for seq, s0, n, _ in merges:
        assert n > 1 and sorted(work[work[:, 0] == seq, 3].tolist()) == list(range(s0, s0 + n))


@settings(max_examples=60, deadline=None, suppress_health_check=[HealthCheck.too_slow])
@given(rows=st.lists(st.tuples(st.integers(0, 1500), st.integers(0, 5000)), min_size=1,
                     max_size=12),
       heads=st.sampled_from(HEADS),
       num_cus=st.sampled_from([0, 1, 64, 256, 1024]))
def test_prefill_plan_properties(rows, heads, num_cus):
    hq, hkv = heads
    q_lens = np.array([q for q, _ in rows], dtype=np.int64)
    kv = np.array([q + p for q, p in rows], dtype=np.int32)
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    info, items, merges = _prefill_plan(q_indptr, kv, hq, hkv, num_cus)
    _check_prefill_plan(q_indptr, q_lens, kv, hq, hkv, info, items, merges)


# ------------------------------------------------------------------------
# Fused page-id space (host-only entry points).

def _desc(num_pages, layers, heads=2, ps=16, d=128, page_stride=None, layer_stride=None):
    slab = heads * ps * d
    ls = slab if layer_stride is None else layer_stride
    return _lib.KVPool(1 << 20, 2 << 20, num_pages, layers * ls if page_stride is None
                       else page_stride, ls, ps * d, d, layers, heads, ps, d, _lib.DTYPE_F16)


@pytest.mark.parametrize("P,N,L,X", [(4, 2, 4, 3), (6, 4, 8, 2), (5, 1, 2, 0), (3, 8, 8, 1)])
def test_fused_pool_and_ids_match_the_oracle_map(P, N, L, X):
    """Page f of the fused pool, local layer j, lies where the oracle's
    fused_slab says the fused id's slab lies in the unfused pool."""
    from oracle import paged_attention_ref as ref

    pool = _desc(P + X, L)
    fused = _lib.KVPool()
    _lib.call("kunserve_fused_pool", ctypes.byref(pool), P, N, ctypes.byref(fused))
    G = L // N
    assert (fused.num_pages, fused.num_layers) == ((P + X) * N, G)
    assert (fused.k, fused.v, fused.layer_stride, fused.head_stride, fused.token_stride) == \
        (pool.k, pool.v, pool.layer_stride, pool.head_stride, pool.token_stride)
    ids = np.arange((P + X) * N, dtype=np.int32)
    pages = np.empty_like(ids)
    _lib.call("kunserve_fused_page_ids", ids.ctypes.data, ids.size, P, N, ids.size,
              pages.ctypes.data)
    for f, page in zip(ids.tolist(), pages.tolist()):
        for j in range(G):
            got = page * fused.page_stride + j * fused.layer_stride
            b, layer = ref.fused_slab(f, j, P, N, L)
            assert got == b * pool.page_stride + layer * pool.layer_stride


def test_fused_helpers_reject_what_they_cannot_map():
    fused = _lib.KVPool()
    layer_major = _desc(8, 4, page_stride=2 * 16 * 128, layer_stride=8 * 2 * 16 * 128)
    with pytest.raises(_lib.KunserveError) as e:
        _lib.call("kunserve_fused_pool", ctypes.byref(layer_major), 8, 2, ctypes.byref(fused))
    assert e.value.code == _lib.EUNSUPPORTED
    with pytest.raises(_lib.KunserveError, match="equal stages"):
        _lib.call("kunserve_fused_pool", ctypes.byref(_desc(8, 6)), 8, 4, ctypes.byref(fused))
    ids = np.array([0, 17], dtype=np.int32)
    out = np.empty_like(ids)
    with pytest.raises(_lib.KunserveError) as e:
        _lib.call("kunserve_fused_page_ids", ids.ctypes.data, 2, 8, 2, 17, out.ctypes.data)
    assert e.value.code == _lib.ERANGE
    ids[1] = -1
    with pytest.raises(_lib.KunserveError):
        _lib.call("kunserve_fused_page_ids", ids.ctypes.data, 2, 8, 2, 17, out.ctypes.data)
