"""Rate-distortion admission (shadowinfer/shadowkv/rd_allocator.py): the
sensitivity proxy and the budget solver.

CPU: the oracle's closed-form ``admit_codes`` (argsort + cumsum +
searchsorted, rd_allocator.py:190-318) is pinned against the known answers of
the reference's own tests (tests/test_rd_allocator.py:64-225,
tests/test_dense_precision.py:255-390) and against an independent
formulation, the one-step-at-a-time greedy loop of ``admit_budget``
(rd_allocator.py:66-170), on random instances with ties, sinks, protected
entries and every budget regime. ``kv_sensitivity`` is pinned against its
definition evaluated with numpy.

GPU: ``si_admit_codes`` / ``si_kv_sensitivity`` through the package API
against the oracle, bit for bit, from tiny shapes to the 8192 x 32 layer.
"""

import numpy as np
import pytest
import torch

from helpers import DT, to_np
from oracle import oracle as O

NAMES = O.CODE_NAMES


def _uniform_map(S, H, p="fp32"):
    return {t: {h: p for h in range(H)} for t in range(S)}


def _map_to_codes(m, S, H):
    return np.array([[O.CODES[m.get(t, {}).get(h, "fp16")] for h in range(H)] for t in range(S)],
                    np.int8)


def _codes_to_map(c):
    return {t: {h: NAMES[int(x)] for h, x in enumerate(row)} for t, row in enumerate(c)}


# ------------------------------------------------------------------ oracle (CPU)
def test_entry_bytes_known_answers():
    """tests/test_rd_allocator.py:64-72."""
    assert O.entry_bytes("fp32", 2, 16) == 2 * 2 * 16 * 4
    assert O.entry_bytes("fp16", 2, 16) == 2 * 2 * 16 * 2
    assert O.entry_bytes("int8", 2, 16) == 2 * (2 * 16 + 2 * 4)
    assert O.entry_bytes("int4", 2, 16) == 2 * (2 * 16 / 2 + 2 * (16 // 16) * 4)
    assert O.entry_bytes("int4", 2, 48) == 2 * (2 * 48 / 2 + 2 * (48 // 16) * 4)
    assert O.entry_bytes("int4", 2, 20) == 2 * (2 * 20 / 2 + 2 * (20 // 20) * 4)
    assert O.entry_bytes("evicted", 2, 16) == 0
    # every cost is an integer-valued float, so int() per entry == int() of a sum
    for B in (1, 2, 3):
        for D in (15, 16, 45, 64):
            for p in ("fp32", "fp16", "int8", "int4"):
                assert float(O.entry_bytes(p, B, D)).is_integer()


def test_oracle_sensitivity_matches_definition():
    """tests/test_rd_allocator.py:75-90, plus the bf16/fp16 rounding of every op."""
    rng = np.random.default_rng(901)
    k = rng.standard_normal((2, 3, 5, 16)).astype(np.float32)
    v = rng.standard_normal((2, 3, 5, 16)).astype(np.float32)
    got = O.kv_sensitivity(k, v, O.F32)
    want = np.zeros((5, 3), np.float32)
    for t in range(5):
        for h in range(3):
            ka = np.abs(k[:, h, t, :]).max()
            va = np.abs(v[:, h, t, :]).max()
            want[t, h] = (ka * ka + va * va) / np.float32(2.0)
    np.testing.assert_array_equal(got, want)
    # bf16: torch rounds the square, the sum and the halving to bf16
    kb = torch.from_numpy(k).to(torch.bfloat16)
    vb = torch.from_numpy(v).to(torch.bfloat16)
    ref = ((kb.abs().amax(dim=(0, -1)).square() + vb.abs().amax(dim=(0, -1)).square()) / 2.0)
    ref = ref.transpose(0, 1).contiguous()
    got = O.kv_sensitivity(to_np(kb), to_np(vb), O.BF16)
    np.testing.assert_array_equal(got, to_np(ref))
    # NaN propagates through the max
    k[0, 1, 2, 3] = np.nan
    assert np.isnan(O.kv_sensitivity(k, v, O.F32)[2, 1])


def _ut9(imp, sens, S, budget, sink=0, rd=True, evict=False, protected=None):
    m = _uniform_map(S, 1)
    prot = None
    if protected:
        prot = np.zeros((S, 1), bool)
        for t, h in protected:
            prot[t, h] = True
    codes, pred, ev = O.admit_codes(_map_to_codes(m, S, 1), imp, sens, budget, 1, 16, sink, rd,
                                    evict, prot)
    greedy = O.admit_budget_greedy(imp, sens, m, budget, 1, 16, sink, rd, evict, protected)
    assert (_codes_to_map(codes), pred, ev) == greedy
    return [NAMES[int(c)] for c in codes[:, 0]], pred, ev


def test_oracle_known_answers_reference_scenarios():
    """The expectations of tests/test_rd_allocator.py:93-225."""
    d = int(O.entry_bytes("fp32", 1, 16)) - int(O.entry_bytes("fp16", 1, 16))
    # UT-9.3: rd ordering downgrades the lowest-sensitivity entry first
    got, pred, ev = _ut9(np.ones((4, 1)), np.array([[9.0], [0.1], [0.5], [1.0]]), 4, 512 - d, sink=1)
    assert got == ["fp32", "fp16", "fp32", "fp32"] and ev == 0 and pred <= 512 - d
    # UT-9.4: importance ordering when rd is off
    got, pred, ev = _ut9(np.array([[0.1], [0.2], [0.3], [0.4]]), np.ones((4, 1)), 4, 512 - d, rd=False)
    assert got[:2] == ["fp16", "fp32"] and ev == 0
    # UT-9.5: protected entries are never touched; the rest are evicted
    got, pred, ev = _ut9(np.full((4, 1), 0.5), np.ones((4, 1)), 4, 0, sink=1, evict=True,
                         protected={(2, 0)})
    assert got == ["fp32", "evicted", "fp32", "evicted"] and ev == 2
    assert pred == int(O.entry_bytes("fp32", 1, 16)) * 2
    # UT-9.6: hard eviction meets a tiny budget
    got, pred, ev = _ut9(np.full((4, 1), 0.5), np.ones((4, 1)), 4, 1, evict=True)
    assert got == ["evicted"] * 4 and pred == 0 and ev > 0
    # UT-9.7: without eviction the int4 floor stays over budget
    got, pred, ev = _ut9(np.full((3, 1), 0.5), np.ones((3, 1)), 3, 1)
    assert got == ["int4"] * 3 and ev == 0 and pred == 3 * int(O.entry_bytes("int4", 1, 16))


def _random_case(rng, S, H, ties=False):
    if ties:
        imp = rng.integers(0, 4, size=(S, H)).astype(np.float32) / 4
        sens = np.ones((S, H), np.float32)
    else:
        imp = rng.random((S, H)).astype(np.float32)
        sens = (rng.random((S, H)) * 5.0).astype(np.float32)
    codes = rng.integers(0, 5, size=(S, H)).astype(np.int8)
    prot = rng.random((S, H)) < 0.1
    return codes, imp, sens, prot


@pytest.mark.parametrize("seed", range(6))
def test_oracle_closed_form_matches_greedy_loop(seed):
    """admit_codes == admit_budget on the same instances (the equivalence the
    reference asserts in tests/test_dense_precision.py:255-370), over random
    codes, ties, sinks, protection and every budget regime."""
    rng = np.random.default_rng(seed)
    S, H, B, D = int(rng.integers(3, 24)), int(rng.integers(1, 5)), int(rng.integers(1, 3)), 16
    codes, imp, sens, prot = _random_case(rng, S, H, ties=seed % 2 == 1)
    costs = O.code_costs(B, D)
    total = int(costs[codes.astype(np.int64)].sum())
    pset = {(int(t), int(h)) for t, h in zip(*np.nonzero(prot))}
    m = _codes_to_map(codes)
    for budget in (None, -1, 0, 1, total // 3, total // 2, total - 1, total, total + 5):
        for rd in (True, False):
            for evict in (False, True):
                sink = int(rng.integers(0, 3))
                got = O.admit_codes(codes, imp, sens, budget, B, D, sink, rd, evict, prot)
                want = O.admit_budget_greedy(imp, sens, m, budget, B, D, sink, rd, evict, pset)
                assert (_codes_to_map(got[0]), got[1], got[2]) == want, (budget, rd, evict, sink)
                np.testing.assert_array_equal(codes, _map_to_codes(m, S, H))  # not mutated


def test_oracle_all_ties_follow_index_order():
    """tests/test_dense_precision.py:329-351: equal scores rank token-major."""
    S, H = 8, 3
    m = _uniform_map(S, H)
    imp = np.full((S, H), 0.5, np.float32)
    one = np.ones((S, H), np.float32)
    got = O.admit_codes(_map_to_codes(m, S, H), imp, one, 1, 1, 16, 0, True, True)
    assert (_codes_to_map(got[0]), got[1], got[2]) == O.admit_budget_greedy(imp, one, m, 1, 1, 16,
                                                                            allow_eviction=True)
    # a budget that cuts mid-list: the first entries in index order go first
    c = O.code_costs(1, 16)
    budget = S * H * int(c[0]) - 5 * int(c[0] - c[3]) - 1
    out, _, _ = O.admit_codes(_map_to_codes(m, S, H), imp, one, budget, 1, 16)
    flat = out.reshape(-1)
    assert list(flat[:5]) == [3] * 5 and flat[5] != 0 and (flat[6:] == 0).all()


# ------------------------------------------------------------------ HIP (GPU)
def _dev_admit(dev, codes, imp, sens, budget, B, D, sink, rd, evict, prot):
    from shadowinfer_amd.shadowkv import admit_codes
    c = torch.from_numpy(codes).to(dev)
    out, pred, ev = admit_codes(c, torch.from_numpy(imp), torch.from_numpy(sens), budget, B, D,
                                sink, rd, evict, None if prot is None else torch.from_numpy(prot))
    assert out.dtype == torch.int8 and out.device == c.device
    assert torch.equal(c.cpu(), torch.from_numpy(codes))  # input not mutated
    return out.cpu().numpy(), pred, ev


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(2, 3, 5, 16), (1, 4, 37, 48), (2, 2, 9, 45), (3, 5, 130, 64)])
def test_hip_sensitivity_bit_exact(dev, dtype, shape):
    from shadowinfer_amd.shadowkv import kv_sensitivity
    g = torch.Generator().manual_seed(sum(shape))
    k = (torch.randn(shape, generator=g) * 3).to(dtype)
    v = (torch.randn(shape, generator=g) * 3).to(dtype)
    got = kv_sensitivity(k.to(dev), v.to(dev))
    assert got.shape == (shape[2], shape[1]) and got.dtype == dtype
    np.testing.assert_array_equal(to_np(got), O.kv_sensitivity(to_np(k), to_np(v), DT[dtype]))


@pytest.mark.gpu
def test_hip_sensitivity_layer_and_nan(dev):
    from shadowinfer_amd.shadowkv import kv_sensitivity
    g = torch.Generator(device=dev).manual_seed(5)
    k = torch.randn(1, 32, 8192, 128, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(1, 32, 8192, 128, generator=g, device=dev).to(torch.bfloat16)
    got = to_np(kv_sensitivity(k, v))
    np.testing.assert_array_equal(got, O.kv_sensitivity(to_np(k), to_np(v), O.BF16))
    k[0, 7, 100, 3] = float("nan")
    got = kv_sensitivity(k, v).float().cpu()
    assert torch.isnan(got[100, 7]) and not torch.isnan(got[101, 7])


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(8))
def test_hip_admit_codes_matches_oracle(dev, seed):
    rng = np.random.default_rng(100 + seed)
    S, H = [(6, 2), (8, 3), (64, 8), (512, 8), (300, 7), (1, 1), (2049, 3), (97, 32)][seed]
    B, D = 1 + seed % 2, 16 if seed % 3 else 48
    codes, imp, sens, prot = _random_case(rng, S, H, ties=seed % 2 == 0)
    total = int(O.code_costs(B, D)[codes.astype(np.int64)].sum())
    for budget in (None, 0, 1, total // 4, total // 2, total - 1, total, 2 * total):
        for rd, evict, sink in ((True, False, 0), (False, True, 2), (True, True, 1)):
            p = prot if sink == 1 else None
            want = O.admit_codes(codes, imp, sens, budget, B, D, sink, rd, evict, p)
            got = _dev_admit(dev, codes, imp, sens, budget, B, D, sink, rd, evict, p)
            np.testing.assert_array_equal(got[0], want[0], err_msg=f"{budget} {rd} {evict}")
            assert got[1:] == want[1:], (budget, rd, evict, sink)


@pytest.mark.gpu
def test_hip_admit_codes_layer_size(dev):
    """The 7B-layer plan (8192 x 32 token-heads), with score ties, NaN, +-0."""
    rng = np.random.default_rng(7)
    S, H, B, D = 8192, 32, 1, 128
    codes = np.ones((S, H), np.int8)
    codes[rng.random((S, H)) < 0.2] = 0
    imp = rng.random((S, H)).astype(np.float32)
    imp[rng.random((S, H)) < 0.3] = 0.25          # many exact ties
    imp[5, 3], imp[9, 1], imp[11, 0] = np.nan, -0.0, 0.0
    sens = (rng.random((S, H)) * 5.0).astype(np.float32)
    total = int(O.code_costs(B, D)[codes.astype(np.int64)].sum())
    for budget, evict in ((total // 2, False), (total // 5, False), (total // 20, True),
                          (total - 12345, False), (0, True)):
        want = O.admit_codes(codes, imp, sens, budget, B, D, 4, True, evict)
        got = _dev_admit(dev, codes, imp, sens, budget, B, D, 4, True, evict, None)
        np.testing.assert_array_equal(got[0], want[0])
        assert got[1:] == want[1:]


@pytest.mark.gpu
def test_hip_admit_budget_dict_matches_greedy(dev):
    from shadowinfer_amd.shadowkv import admit_budget
    rng = np.random.default_rng(3)
    S, H, B, D = 12, 3, 2, 16
    codes, imp, sens, prot = _random_case(rng, S, H)
    full = _codes_to_map(codes)
    partial = {t: {h: p for h, p in m.items() if (t + h) % 4} for t, m in full.items() if t != 5}
    partial[20] = {0: "fp32", 7: "int8"}  # outside the importance window: counted, never touched
    pset = {(1, 1), (4, 0)}
    total = int(O.code_costs(B, D)[codes.astype(np.int64)].sum())
    for m in (full, partial):
        for budget in (None, 0, 1, total // 3, total // 2, total):
            for evict in (False, True):
                want = O.admit_budget_greedy(imp, sens, m, budget, B, D, 1, True, evict, pset)
                got = admit_budget(torch.from_numpy(imp).to(dev), torch.from_numpy(sens), m, budget,
                                   B, D, sink_tokens=1, allow_eviction=evict, protected=pset)
                assert got == want, (budget, evict)


@pytest.mark.gpu
def test_hip_predict_and_guards(dev):
    from shadowinfer_amd.shadowkv import admit_codes, predict_codes_bytes
    rng = np.random.default_rng(11)
    codes = rng.integers(0, 5, size=(33, 5)).astype(np.int8)
    c = torch.from_numpy(codes).to(dev)
    assert predict_codes_bytes(c, 2, 64) == int(O.code_costs(2, 64)[codes.astype(np.int64)].sum())
    with pytest.raises(ValueError):
        admit_codes(c.reshape(-1), torch.ones(1, 1), torch.ones(1, 1), 1, 1, 16)
    bad = c.clone()
    bad[3, 2] = 7
    with pytest.raises(ValueError):
        admit_codes(bad, torch.rand(33, 5), torch.rand(33, 5), 10, 1, 16)
    empty = torch.zeros(0, 4, dtype=torch.int8, device=dev)
    out, pred, ev = admit_codes(empty, torch.zeros(0, 4), torch.zeros(0, 4), 0, 1, 16,
                                allow_eviction=True)
    assert out.shape == (0, 4) and (pred, ev) == (0, 0)
