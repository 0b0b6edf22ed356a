"""Host-side logic of the shim: step arguments -> kv lengths and CSR tables."""
import numpy as np
import pytest

from kunserve_amd import csr_from_lists, kv_lens_for_step
from kunserve_amd import workloads
from oracle import paged_attention_ref as ref


def test_kv_lens_rule_matches_oracle():
    rng = np.random.default_rng(0)
    first = rng.integers(1, 5000, 50)
    ql = rng.integers(1, 600, 50)
    flag = rng.integers(0, 2, 50)
    ql = np.where(flag == 0, 1, ql)
    got = kv_lens_for_step(first, ql, flag)
    assert np.array_equal(got, ref.kv_lens_for_step(first, ql, flag))
    with pytest.raises(ValueError):
        kv_lens_for_step([0], [3], [0])


def test_kv_lens_with_tensor_cores():
    """use_tensor_cores flags every row as prefill (kunserve/request.py:667-670).
    Given the rows' real stages, a decode row (first = prompt_len +
    output_len) keeps kv_len = first, so its token lands at first - 1
    inside ceil(first / bs) blocks (kunserve/block_manager.py:493-500), and
    a chunk row takes first + q_len. Without them, chunks of several tokens
    and a one-token prompt are still prefill; a one-token row past position
    0 is decode only when its page list cannot hold position `first`, else
    it raises. Whole request lifecycles are checked in test_oracle.py."""
    rng = np.random.default_rng(1)
    first = rng.integers(0, 5000, 200)
    ql = np.where(rng.random(200) < 0.5, 1, rng.integers(2, 600, 200))
    stage = np.where(ql == 1, rng.integers(0, 2, 200), 1)
    flag = np.ones(200, dtype=np.int64)
    got = kv_lens_for_step(first, ql, flag, True, stage)
    assert np.array_equal(got, ref.kv_lens_for_step(first, ql, flag, True, stage))
    assert np.array_equal(got, np.where(stage == 1, first + ql, first))
    # the rows' real stages decide when given
    assert kv_lens_for_step([64], [1], [1], True, is_context_stage=[1]).tolist() == [65]
    assert kv_lens_for_step([64], [1], [1], True, is_context_stage=[0]).tolist() == [64]
    with pytest.raises(ValueError, match="exactly one"):
        kv_lens_for_step([64], [5], [1], True, is_context_stage=[0])
    # without them
    assert kv_lens_for_step([0], [1], [1], use_tensor_cores=True).tolist() == [1]
    assert kv_lens_for_step([64], [7], [1], use_tensor_cores=True).tolist() == [71]
    assert kv_lens_for_step([64], [1], [1], True, None, [4], 16).tolist() == [64]
    for pages in (None, [5]):
        with pytest.raises(ValueError, match="is_context_stage"):
            kv_lens_for_step([64], [1], [1], True, None, pages, 16)


def test_llama_op_reference_call_raises_under_tensor_cores():
    """The reference's 13-argument pforward call (kunserve/flash_backend.py:
    2448-2469) with --use-tensor-cores: every row flagged as prefill and no
    is_context_stage. A step with a one-token row the page counts cannot
    settle raises ValueError before any device work; with the rows' real
    stages the same step is prepared (the kv_len rule is checked here, the
    device step in tests/test_gpu_boundary.py)."""
    import torch
    from kunserve_amd import LlamaOp
    from kunserve_amd.paged_kv import decode_rows

    op = LlamaOp(64, 2, 8, 4, 16, 128, 1, 1, 8, 4096, 4096, 1, torch.device("cpu"),
                 use_tensor_cores=True)
    # rows: the one-token tail chunk of a 513-token prompt (first 512, 33
    # pages) and a decode row (first 40, 3 pages)
    first, flags = [512, 40], [1, 1]
    pages = [list(range(33)), [40, 41, 42]]
    with pytest.raises(ValueError, match="is_context_stage"):
        op.pforward(2, 2, 64, 0, 2, [[7], [9]], first, flags, pages, 0, [], [], 0)
    kv = kv_lens_for_step(first, [1, 1], flags, True, [1, 0], [33, 3], 16)
    assert kv.tolist() == [513, 40]
    assert decode_rows(first, [1, 1], flags, True, [1, 0]).tolist() == [False, True]


def test_csr_truncates_and_validates():
    pages = [[5, 6, 7], [1], [2, 3]]
    indptr, indices = csr_from_lists(pages, np.array([17, 16, 3]), 16, 8)
    assert indptr.tolist() == [0, 2, 3, 4]
    assert indices.tolist() == [5, 6, 1, 2]          # rows truncated to ceil(kv/16) pages
    with pytest.raises(ValueError, match="needs 2"):
        csr_from_lists([[1]], np.array([17]), 16, 8)
    with pytest.raises(IndexError):
        csr_from_lists([[8]], np.array([3]), 16, 8)
    with pytest.raises(IndexError):
        csr_from_lists([[-1]], np.array([3]), 16, 8)
    indptr, indices = csr_from_lists([[], [4]], np.array([0, 1]), 16, 8)
    assert indptr.tolist() == [0, 0, 1] and indices.tolist() == [4]


def test_workloads_are_seeded_and_disjoint():
    for make in (workloads.single_layer_decode, workloads.llama2_7b_decode,
                 workloads.llama3_8b_gqa_decode,
                 lambda: workloads.llama2_7b_decode(page_size=256)):
        a, b = make(), make()
        assert np.array_equal(a.kv_len, b.kv_len)
        indptr, indices = a.csr()
        assert np.unique(indices).size == indices.size            # no page shared
        assert indices.max() < a.num_pages
        assert np.array_equal(np.diff(indptr), (a.kv_len + a.page_size - 1) // a.page_size)
    w = workloads.llama2_7b_decode()
    w256 = workloads.llama2_7b_decode(page_size=256)
    assert np.array_equal(w.kv_len, w256.kv_len) and w256.num_pages * 256 == w.num_pages * 16
    assert w.kv_len.min() >= 16 and w.kv_len.max() <= 4096
    # sample median of 64 lognormal(ln 700, 1) draws: 700 within a few standard errors
    assert 450 <= np.median(w.kv_len) <= 1100


def test_prefill_steps_cover_each_prompt_once():
    p = workloads.chunked_prefill()
    done = np.zeros_like(p.prompt_len)
    for rows, ql, kv in p.steps():
        assert np.all(ql <= p.chunk) and np.all(ql >= 1)
        assert np.array_equal(kv, p.prefix_len[rows] + done[rows] + ql)
        done[rows] += ql
    assert np.array_equal(done, p.prompt_len)
    # causal flop count against a brute-force sum on a tiny case
    tiny = workloads.PrefillShape("t", 2, 2, 4, 16, 8, np.array([5]), np.array([3]), 2, [], 0)
    visible = sum(3 + i + 1 for i in range(5))
    assert tiny.causal_flops() == 4 * 2 * 4 * visible


def test_remap_tables_point_at_copies():
    r = workloads.kv_remap()
    src_set = set(r.src.tolist())
    m = dict(zip(r.src.tolist(), r.dst.tolist()))
    for a, b in zip(r.decode.pages, r.decode_remapped.pages):
        assert [m.get(int(x), int(x)) for x in a] == b.tolist()
    allp = np.concatenate(r.decode.pages)
    assert not np.any((allp >= 8192) & (allp < 16384))
    assert any(int(x) in src_set for x in allp)


def test_kept_layers_follow_the_stage_split():
    """kunserve/flash_backend.py:2395,2442-2443: instance r of g runs layers
    [r * L // g, (r + 1) * L // g); pmm_drop drops the others."""
    from kunserve_amd import kept_layers

    assert kept_layers(32, 0, 1) == range(0, 32)
    assert kept_layers(32, 0, 2) == range(0, 16)
    assert kept_layers(32, 1, 2) == range(16, 32)
    assert kept_layers(80, 3, 4) == range(60, 80)
    # every layer is kept by exactly one instance of the group
    for g in (1, 2, 4, 8):
        owners = sorted(l for r in range(g) for l in kept_layers(32, r, g))
        assert owners == list(range(32))
    with pytest.raises(ValueError):
        kept_layers(30, 0, 4)
    with pytest.raises(ValueError):
        kept_layers(32, 2, 2)


def test_pmm_pool_needs_a_gpu_device():
    import torch

    from kunserve_amd import PmmPool

    with pytest.raises(ValueError, match="GPU device"):
        PmmPool(8, 2, 2, 16, 128, 8, device=torch.device("cpu"))


def test_reference_class_names_resolve_to_this_package():
    """kunserve/models.py:52-65 constructs torch.classes.gpt_ops.LlamaOp and
    kunserve/worker.py:673-681 calls torch.ops.swapping_ops.swap: both names
    resolve to this package once it is imported."""
    import torch

    import kunserve_amd

    assert torch.classes.gpt_ops.LlamaOp is kunserve_amd.LlamaOp
    assert hasattr(torch.ops.swapping_ops, "swap")
    with pytest.raises(RuntimeError):   # other gpt_ops names stay native lookups
        torch.classes.gpt_ops.NotAClassOfThisPackage


def test_llama_op_restore_leaves_the_fusion_group():
    """pmm_drop joins a balloon group (fused page ids); pmm_restore leaves it,
    as restore_from_fusion resets the fusion size
    (kunserve/block_manager.py:347-348), also for an op without extend
    memory, whose drop and restore move no pages."""
    import torch
    from kunserve_amd import LlamaOp

    op = LlamaOp(16, 4, 8, 2, 16, 128, 1, 1, 8, 4096, 4096, 1, torch.device("cpu"))
    assert op.pmm_drop(1, 2) == 0 and op.fusion_size == 2
    assert op.pmm_restore() == [] and op.fusion_size == 1
