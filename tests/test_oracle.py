"""Pins the CPU oracle against the reference's known answers (CPU only).

Each oracle function is checked against vectors from the reference's own
tests (tests/golden/reference_kats.json), hand-derived values, closed forms
or an independent formulation -- never against a retyped copy of itself.
A planted-mistake test shows the checks would catch a wrong oracle.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import lora as olora
from oracle import mapping as omap


# -- promote_rank ------------------------------------------------------------
def test_promote_rank_table(kats):
    k = kats["promote_rank"]
    for rank, expected in k["cases"]:
        assert omap.promote_rank(rank) == expected
    for r in omap.SUPPORTED_RANKS:
        assert omap.promote_rank(r) == r
    for r in k["unchanged"]:
        assert omap.promote_rank(r) == r
    for r in k["raises"]:
        with pytest.raises(ValueError):
            omap.promote_rank(r)


# -- latest-wins routing -----------------------------------------------------
def _layout(kats, name):
    return kats["latest_wins"][name]


def test_latest_wins_cases(kats):
    for case in kats["latest_wins"]["cases"]:
        atok = _layout(kats, case["layout"])
        got = omap.latest_wins_ids(case["tokens"], atok, base_reset=case["layout"] == "base_reset")
        assert got == case["expected"], case


def test_latest_wins_chunked(kats):
    for case in kats["latest_wins"]["chunked"]["cases"]:
        atok = _layout(kats, case["layout"])
        out, cur, off = [], 0, 0
        for n in case["chunks"]:
            part = omap.latest_wins_ids(case["tokens"][off:off + n], atok, case["layout"] == "base_reset", cur)
            out += part
            cur = part[-1]
            off += n
        assert out == case["expected"], case


def test_alora_gating_is_latest_wins_with_one_control_token():
    """Gating by an activation offset == latest-wins with a control token there."""
    rng = np.random.default_rng(3)
    lens = [5, 17, 1, 40]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    adapters = [3, 1, 2, 4]
    offs = np.array([2, 0, 5, 39])
    cached = np.array([0, 10, 4, 0])          # chunked prefill: absolute positions
    req = np.repeat(adapters, lens)
    pos = np.concatenate([c + np.arange(l) for c, l in zip(cached, lens)])
    got = omap.alora_effective_ids(req, pos, cu, offs)
    for s, (l, a) in enumerate(zip(lens, adapters)):
        full_len = cached[s] + l
        text, ctl = 50, 100 + a
        seq = [ctl if q == offs[s] else text for q in range(full_len)]
        atok = [101, 102, 103, 104]
        exp = omap.latest_wins_ids(seq, atok, base_reset=False)[cached[s]:]
        assert list(got[cu[s]:cu[s + 1]]) == exp
    _ = rng


# -- remap / finalize tables -------------------------------------------------
def test_remap_non_applicable_and_stable_rank_sort():
    # adapters (0-based): ranks 32, 8(->16), 0 (n/a), 16, 32 ; adapter 4 all-zero A
    ranks = [32, 8, 16, 16, 32]
    applicable = [True, True, False, True, False]
    remap, order, eff = omap.build_remap(applicable, ranks)
    # promoted ranks 32,16,16,16,32; applicable 0,1,3 -> stable sort by rank: 1,3 (16) then 0 (32)
    assert order == [1, 3, 0]
    assert remap.tolist() == [0, 3, 1, 0, 2, 0]
    assert eff == [32, 16, 16, 16, 32]


def test_finalize_tables_hand_values():
    # QKV-like slices (64, 32, 32), block_n 32; applicable adapters: two tier-16, one tier-32
    order, eff = [1, 3, 0], [32, 16, 16, 16]
    na, tile_slice, scr, tiers = omap.finalize_tables((64, 32, 32), order, eff, block_n=32)
    assert na == (2, 1, 0, 0, 0, 0)
    assert tile_slice.tolist() == [0, 0, 1, 2]
    # N_total = 128; tier16 base 128, tier32 base 128 + 2*3*16 = 224, tier64.. base 224 + 1*3*32 = 320
    assert scr.tolist() == [[128, 224, 320, 320, 320, 320],
                            [144, 256, 384, 448, 576, 832],
                            [160, 288, 448, 576, 832, 1344]]
    assert tiers == {16: [1, 3], 32: [0]}
    with pytest.raises(AssertionError):
        omap.finalize_tables((48, 32), order, eff, block_n=32)


# -- bitmasks ----------------------------------------------------------------
def test_bitmask_hand_derived(kats):
    k = kats["bitmask"]
    remap_t = np.array(k["remap_tables"]).T
    for bm, expected in k["hand_derived"].items():
        got = omap.compute_bitmasks(k["adapter_indices"], remap_t, int(bm))
        assert got.tolist() == expected, bm
    # block_m = 1: each token's own bit
    got1 = omap.compute_bitmasks(k["adapter_indices"], remap_t, 1)
    for m, table in enumerate(k["remap_tables"]):
        exp = [(1 << (table[i] - 1)) if table[i] > 0 else 0 for i in k["adapter_indices"]]
        assert got1[m].tolist() == exp


@pytest.mark.parametrize("block_m", [1, 8, 16, 32, 64])
def test_bitmask_unit_cases(block_m):
    """The literal asserts of tests/unit/test_bitmask_computation.py:30-184."""
    t = lambda tables: np.array(tables).T
    assert omap.compute_bitmasks(np.ones(block_m, int), t([[0, 1]]), block_m).tolist() == [[1]]
    if block_m >= 2:
        half = block_m // 2
        ids = np.concatenate([np.ones(half, int), np.full(block_m - half, 2)])
        assert omap.compute_bitmasks(ids, t([[0, 1, 2]]), block_m).tolist() == [[3]]
    assert omap.compute_bitmasks(np.zeros(block_m, int), t([[0, 1, 2]]), block_m).tolist() == [[0]]
    assert omap.compute_bitmasks(np.full(block_m, 2), t([[0, 1, 0]]), block_m).tolist() == [[0]]
    assert omap.compute_bitmasks(np.ones(block_m, int), t([[0, 1, 0], [0, 0, 1]]), block_m).tolist() == [[1], [0]]
    ids = np.concatenate([np.ones(block_m, int), np.full(block_m, 2)])
    assert omap.compute_bitmasks(ids, t([[0, 1, 2]]), block_m).tolist() == [[1, 2]]
    if block_m > 1:
        ids = np.concatenate([np.ones(block_m, int), np.zeros(1, int)])
        assert omap.compute_bitmasks(ids, t([[0, 1, 2]]), block_m).tolist() == [[1, 0]]


def test_bitmask_sign_bit():
    remap_t = np.arange(65).reshape(1, 65).T
    got = omap.compute_bitmasks([64, 1], remap_t, 32)
    assert got[0, 0] == np.int64(-(2 ** 63)) | 1
    assert got[0, 0] < 0


def test_remapped_indices():
    tables = [[0, 1, 2, 3, 4], [0, 1, 0, 2, 0], [0, 3, 1, 2, 0]]
    ids = [0, 4, 2, 1, 3]
    got = omap.remapped_indices(ids, np.array(tables).T)
    assert got.tolist() == [[tables[m][i] for i in ids] for m in range(3)]


# -- segments ----------------------------------------------------------------
def test_segments_brute_force():
    rng = np.random.default_rng(0)
    for trial in range(50):
        NA = int(rng.integers(1, 30))
        T = int(rng.integers(0, 300))
        ids = rng.integers(-2, NA + 3, size=T)
        seg, perm = omap.build_segments(ids, NA)
        valid = (ids >= 1) & (ids <= NA)
        assert seg[0] == 0 and seg[-1] == valid.sum() == perm.size
        for g in range(1, NA + 1):
            toks = perm[seg[g - 1]:seg[g]]
            assert list(toks) == [t for t in range(T) if ids[t] == g]   # grouped, ascending


# -- switched-LoRA math ------------------------------------------------------
def test_identity_closed_form(kats):
    k = kats["lora_identity"]
    IN, OUT, R = k["in_features"], k["out_features"], k["rank"]
    NA = 4
    A = np.zeros((NA, 1, R, IN))
    B = np.zeros((NA, 1, OUT, R))
    for a in range(NA):
        A[a, 0] = np.eye(R, IN) * 0.1 * (a + 1)
        B[a, 0] = np.eye(OUT, R) * 0.2 * (a + 1)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((12, IN))
    y = rng.standard_normal((12, OUT))
    ids = np.array([0, 1, 2, 3, 4, 0, 4, 3, 2, 1, 1, 0])
    got = olora.switched_lora_apply(y, x, ids, [A], [B], (OUT,), dtype="f64")
    exp = y.copy()
    for t, a in enumerate(ids):
        if a:
            exp[t, :R] += x[t, :R] * 0.02 * a * a
    np.testing.assert_allclose(got, exp, rtol=1e-12, atol=1e-12)


def test_switched_math_matches_per_token_loop():
    rng = np.random.default_rng(2)
    NA, H, slices, maxr = 5, 24, (16, 8, 8), 12
    ranks = [4, 12, 8, 1, 12]
    A = [rng.standard_normal((NA, 1, maxr, H)) for _ in slices]
    B = [rng.standard_normal((NA, 1, o, maxr)) for o in slices]
    for s in range(len(slices)):
        for a in range(NA):
            A[s][a, 0, ranks[a]:] = 0
            B[s][a, 0, :, ranks[a]:] = 0
    x = rng.standard_normal((30, H))
    y = rng.standard_normal((30, sum(slices)))
    ids = rng.integers(0, NA + 1, size=30)
    got = olora.switched_lora_apply(y, x, ids, A, B, slices, ranks, dtype="f64")
    exp = olora.per_token_reference(y, x, ids, A, B, slices, ranks)
    np.testing.assert_allclose(got, exp, rtol=1e-12, atol=1e-12)
    # base rows are returned untouched
    assert np.array_equal(got[ids == 0], y[ids == 0])


def test_bf16_round_known_values():
    vals = np.array([1.0, 1.00390625, 1.005859375, 1.0078125, 3.14159265, -2.5e-3, 65504.0], dtype=np.float32)
    # 1 + 2^-8 is a tie between 1 and 1+2^-7 -> even (1.0); 1.005859375 rounds up
    exp = np.array([1.0, 1.0, 1.0078125, 1.0078125, 3.140625, -0.0025024414, 65536.0], dtype=np.float32)
    np.testing.assert_array_equal(olora.bf16_round(vals), exp)


def _xext_setup(slices, seed):
    rng = np.random.default_rng(seed)
    NA, H = 4, 32
    adapter_ranks = [16, 8, 32, 16]
    A = [rng.standard_normal((NA, 1, 32, H)) for _ in slices]
    B = [rng.standard_normal((NA, 1, o, 32)) for o in slices]
    for s in range(len(slices)):
        for a in range(NA):
            A[s][a, 0, adapter_ranks[a]:] = 0
            B[s][a, 0, :, adapter_ranks[a]:] = 0
    applicable = omap.applicability(A, adapter_ranks)
    remap, order, eff = omap.build_remap(applicable, adapter_ranks)
    na, tile_slice, scr, tiers = omap.finalize_tables(slices, order, eff, 32)
    W = rng.standard_normal((sum(slices), H))
    w_ext = omap.build_w_ext(W, A, tiers)
    lb = omap.build_lb_packed(B, tiers)
    x = rng.standard_normal((40, H))
    ids = rng.integers(0, NA + 1, size=40)
    loc = remap[ids]
    bm = omap.compute_bitmasks(loc, np.arange(NA + 1).reshape(-1, 1), 32)[0]
    exp = olora.switched_lora_apply(x @ W.T, x, ids, A, B, slices, adapter_ranks, dtype="f64")
    return dict(x_ext=x @ w_ext.T, loc=loc, bm=bm, lb=lb, tile_slice=tile_slice, scr=scr, na=na, exp=exp)


def test_xext_expand_equals_switched_math():
    """expand over x_ext = x . w_ext^T reproduces base + delta (fp64, no rounding)."""
    slices = (64, 32)
    d = _xext_setup(slices, 4)
    got = olora.switch_lora_expand_xext(d["x_ext"], d["loc"], d["bm"], d["lb"], d["tile_slice"], d["scr"], d["na"],
                                        len(slices), 32, sum(slices), dtype="f64")[:, :sum(slices)]
    np.testing.assert_allclose(got, d["exp"], rtol=1e-10, atol=1e-10)


def test_xext_swiglu_equals_silu_of_corrected_output():
    """The SwiGLU epilogue is silu(g)*u of exactly the corrected gate/up."""
    slices = (32, 32)
    d = _xext_setup(slices, 5)
    sw = olora.expand_swiglu_xext(d["x_ext"], d["loc"], d["bm"], d["lb"], d["scr"], d["na"], 2, 32, 64, dtype="f64")
    g, u = d["exp"][:, :32], d["exp"][:, 32:64]
    np.testing.assert_allclose(sw, g / (1 + np.exp(-g)) * u, rtol=1e-10, atol=1e-10)


def test_swiglu_hand_values():
    # one row, no adapter: out = silu(g) * u with g = 0 -> 0, g = 2, u = 3 -> 2/(1+e^-2)*3
    xe = np.zeros((1, 64))
    xe[0, 1] = 2.0
    xe[0, 32 + 1] = 3.0
    out = olora.expand_swiglu_xext(xe, [0], [0], np.zeros(1), np.zeros((2, 6), np.int32), (0,) * 6, 2, 32, 64,
                                   dtype="f64")
    assert out[0, 0] == 0.0
    assert abs(out[0, 1] - 2.0 / (1.0 + np.exp(-2.0)) * 3.0) < 1e-12


def test_planted_mistake_is_caught(monkeypatch):
    """A transposed-operand mistake in the oracle fails the identity closed form."""
    real = olora.switched_lora_apply

    def wrong(y, x, ids, A_sl, B_sl, slices, ranks=None, dtype="bf16", mode="exact"):
        A_bad = [np.flip(np.asarray(a), axis=2).copy() for a in A_sl]   # wrong rank-row order
        return real(y, x, ids, A_bad, B_sl, slices, ranks, dtype, mode)

    monkeypatch.setattr(olora, "switched_lora_apply", wrong)
    with pytest.raises(AssertionError):
        test_identity_closed_form({"lora_identity": {"in_features": 32, "out_features": 16, "rank": 8}})


# -- applicability -------------------------------------------------------------
def test_applicability_hand_cases():
    """src/granite_switch/vllm/core/lora.py:353-362: any nonzero value in the
    first r rows of lora_A, in any slice, makes an adapter applicable."""
    NA, maxr, H = 5, 8, 6
    A0 = np.zeros((NA, 1, maxr, H))
    A1 = np.zeros((NA, 1, maxr, H))
    A0[0, 0, 3, 2] = 1.0          # adapter 0: nonzero inside its rank (4) in slice 0
    A0[1, 0, 5, 0] = 2.0          # adapter 1: nonzero only in row 5, past its rank (4)
    A1[2, 0, 0, 5] = -1.0         # adapter 2: zero in slice 0, nonzero in slice 1
    A0[3, 0, 0, 0] = 1.0          # adapter 3: rank 0 never applies
    ranks = [4, 4, 4, 0, 8]       # adapter 4: all zero
    assert omap.applicability([A0, A1], ranks) == [True, False, True, False, False]
    # rank past the nonzero row: adapter 1 at rank 6 applies
    assert omap.applicability([A0, A1], [4, 6, 4, 0, 8])[1] is True


# -- probe routing -------------------------------------------------------------
def test_probe_kind_lut_kats(kats):
    for case in kats["probe_routing"]["lut_cases"]:
        lut = omap.build_adapter_kind_lut(case["adapter_kinds"])
        if case["lut"] is None:
            assert lut is None
        else:
            assert lut.tolist() == case["lut"]


def test_split_adapter_indices_kats(kats):
    for case in kats["probe_routing"]["split_cases"]:
        lut = omap.build_adapter_kind_lut(case["adapter_kinds"])
        lora, probe = omap.split_adapter_indices(lut, case["ids"])
        assert lora.tolist() == case["lora"], case
        assert probe.tolist() == case["probe"], case


def test_split_adapter_indices_partition():
    """Every index lands in exactly one stream; probe streams hold only probe slots."""
    rng = np.random.default_rng(9)
    lut = omap.build_adapter_kind_lut(["lora", "probe", "lora", "probe", "probe"])
    ids = rng.integers(0, 6, size=(7, 33))
    lora, probe = omap.split_adapter_indices(lut, ids)
    assert np.array_equal(lora + probe, ids)
    assert np.all((lora == 0) | (probe == 0))
    assert set(np.unique(probe).tolist()) <= {0, 2, 4, 5}
    assert set(np.unique(lora).tolist()) <= {0, 1, 3}


# -- shrink rows ---------------------------------------------------------------
def test_shrink_rows_identity_closed_form():
    """With A_a = eye(r, H) * 0.1 (a+1) (tests/shared/lora_cases.py:355-426),
    slot k of adapter a holds 0.1 (a+1) x[perm[k], :r] in every slice."""
    rng = np.random.default_rng(4)
    NA, H, maxr, S = 4, 20, 8, 3
    ranks = [8, 4, 0, 6]
    A = []
    for s in range(S):
        a_s = np.zeros((NA, 1, maxr, H))
        for a in range(NA):
            a_s[a, 0, :ranks[a]] = np.eye(ranks[a], H) * 0.1 * (a + 1)
        A.append(a_s)
    T = 30
    x = rng.standard_normal((T, H))
    ids = rng.integers(0, NA + 1, size=T)
    seg, perm = omap.build_segments(ids, NA)
    z = olora.shrink_rows(x, perm, seg, A, ranks, S * maxr)
    for g in range(1, NA + 1):
        r = ranks[g - 1]
        for k in range(seg[g - 1], seg[g]):
            t = perm[k]
            for s in range(S):
                exp = 0.1 * g * x[t, :r]
                np.testing.assert_allclose(z[k, s * r:(s + 1) * r], exp, rtol=1e-12, atol=1e-12)
            assert np.all(z[k, S * r:] == 0)


def test_per_token_reference_identity_closed_form(kats):
    k = kats["lora_identity"]
    IN, OUT, R, NA = k["in_features"], k["out_features"], k["rank"], 4
    A = np.zeros((NA, 1, R, IN))
    B = np.zeros((NA, 1, OUT, R))
    for a in range(NA):
        A[a, 0] = np.eye(R, IN) * 0.1 * (a + 1)
        B[a, 0] = np.eye(OUT, R) * 0.2 * (a + 1)
    rng = np.random.default_rng(6)
    x = rng.standard_normal((9, IN))
    y = rng.standard_normal((9, OUT))
    ids = np.array([4, 0, 1, 2, 3, 3, 0, 1, 4])
    got = olora.per_token_reference(y, x, ids, [A], [B], (OUT,), [R] * NA)
    exp = y.copy()
    for t, a in enumerate(ids):
        if a:
            exp[t, :R] += x[t, :R] * 0.02 * a * a
    np.testing.assert_allclose(got, exp, rtol=1e-12, atol=1e-12)


# -- the CPU baseline loop -----------------------------------------------------
def _hf_case(dtype, seed):
    import torch

    rng = np.random.default_rng(seed)
    NA, H, slices, maxr = 5, 48, (32, 16, 16), 16
    ranks = [16, 8, 0, 12, 16]
    A = [rng.standard_normal((NA, 1, maxr, H)) / np.sqrt(H) for _ in slices]
    B = [rng.standard_normal((NA, 1, o, maxr)) * 0.5 for o in slices]
    for s in range(len(slices)):
        for a in range(NA):
            A[s][a, 0, ranks[a]:] = 0
            B[s][a, 0, :, ranks[a]:] = 0
    x = rng.standard_normal((40, H))
    y = rng.standard_normal((40, sum(slices)))
    ids = rng.integers(0, NA + 1, size=40)
    ids[:3] = 0
    to = lambda a: torch.tensor(a, dtype=dtype)
    if dtype != torch.float64:
        # inputs representable in the dtype, so both sides start from the same values
        x, y = to(x).double().numpy(), to(y).double().numpy()
        A = [to(a).double().numpy() for a in A]
        B = [to(b).double().numpy() for b in B]
    return dict(x=x, y=y, ids=ids, A=A, B=B, slices=slices, ranks=ranks, to=to)


def test_hf_loop_matches_oracle_f64():
    """The baseline loop and the oracle agree exactly in float64."""
    import torch

    from oracle import baseline

    c = _hf_case(torch.float64, 11)
    out = c["to"](c["y"])
    baseline.hf_loop(out, c["to"](c["x"]), torch.tensor(c["ids"]), [c["to"](a) for a in c["A"]],
                     [c["to"](b) for b in c["B"]], c["slices"])
    exp = olora.switched_lora_apply(c["y"], c["x"], c["ids"], c["A"], c["B"], c["slices"], c["ranks"], dtype="f64")
    np.testing.assert_allclose(out.numpy(), exp, rtol=1e-12, atol=1e-12)
    assert np.array_equal(out.numpy()[c["ids"] == 0], c["y"][c["ids"] == 0])


@pytest.mark.parametrize("name,tol", [("bfloat16", 2e-2), ("float32", 1e-5)])
def test_hf_loop_matches_oracle_rounding_mode(name, tol):
    """In bf16 / fp32 the loop follows the oracle's "hf" rounding sequence
    (shrink rounded, expand rounded, then the add rounded)."""
    import torch

    from oracle import baseline

    dt = getattr(torch, name)
    c = _hf_case(dt, 12)
    out = c["to"](c["y"])
    baseline.hf_loop(out, c["to"](c["x"]), torch.tensor(c["ids"]), [c["to"](a) for a in c["A"]],
                     [c["to"](b) for b in c["B"]], c["slices"])
    dname = "bf16" if dt == torch.bfloat16 else "fp32"
    exp = olora.switched_lora_apply(c["y"], c["x"], c["ids"], c["A"], c["B"], c["slices"], c["ranks"], dtype=dname,
                                    mode="hf")
    got = out.double().numpy()
    assert np.all(np.abs(got - exp) <= tol + tol * np.abs(exp))
    assert np.array_equal(got[c["ids"] == 0], c["y"][c["ids"] == 0])


# -- W-less shrink-expand ------------------------------------------------------
def _wless_case(adapters_spec, ids, K, N, seed):
    """Packed metadata built by hand, as tests/unit/test_wcross_shrink_kernel.py:41-101
    does it, independently of finalize_tables: adapters in ascending rank
    order, kernel-local ids 1.. in that order, no base rows in the cross
    weight, so shrink columns start at 0."""
    rng = np.random.default_rng(seed)
    adapters = [(r, rng.standard_normal((r, K)) * 0.05, rng.standard_normal((N, r)) * 0.05) for r in adapters_spec]
    w_ext = np.concatenate([A for _, A, _ in adapters], axis=0)
    na = tuple(sum(1 for r, _, _ in adapters if r == R) for R in omap.SUPPORTED_RANKS)
    slice_col = np.zeros((1, 6), dtype=np.int32)
    running = 0
    for k_, R in enumerate(omap.SUPPORTED_RANKS):
        slice_col[0, k_] = running
        running += na[k_] * R
    lb = np.concatenate([np.stack([B for r, _, B in adapters if r == R]).reshape(-1)
                         for R in omap.SUPPORTED_RANKS if any(r == R for r, _, _ in adapters)])
    col_of = np.cumsum([0] + [r for r, _, _ in adapters])[:-1]
    ids = np.asarray(ids)
    M = ids.shape[0]
    x = rng.standard_normal((M, K))
    x_ext = x @ w_ext.T
    bm = np.zeros((M + 31) // 32, dtype=np.int64)
    for m, a in enumerate(ids):
        if a > 0:
            bm[m // 32] |= np.int64(1) << np.int64(a - 1)
    ref = np.zeros((M, N))
    for m, a in enumerate(ids):
        if a > 0:
            r, _, B = adapters[a - 1]
            ref[m] = x_ext[m, col_of[a - 1]:col_of[a - 1] + r] @ B.T
    return dict(x_ext=x_ext, ids=ids, bm=bm, lb=lb, tile_slice=np.zeros(N // 32, np.int32), scr=slice_col, na=na,
                ref=ref)


@pytest.mark.parametrize("spec,ids,K,N", [
    ((16,), [0, 1] * 20, 256, 64),                      # single tier, mixed rows, two row tiles
    ((16,), [0] * 32, 256, 64),                         # one all-base tile
    ((16, 32), [0, 1, 2, 2, 0, 1] * 8, 512, 128),       # two tiers
    ((16, 16), [1, 2, 0, 1, 2, 0] * 8, 256, 64),        # two adapters of one tier
    ((16, 32, 64), [3] * 5 + [0] * 40 + [1, 2] * 10, 128, 96),
])
def test_shrink_expand_xext_matches_per_token_loop(spec, ids, K, N):
    d = _wless_case(spec, ids, K, N, seed=len(ids) + K)
    got = olora.shrink_expand_xext(d["x_ext"], d["ids"], d["bm"], d["lb"], d["tile_slice"], d["scr"], d["na"], 1, 32,
                                   N, dtype="f64")
    np.testing.assert_allclose(got, d["ref"], rtol=1e-10, atol=1e-12)
    base = d["ids"] == 0
    assert np.all(got[base] == 0)                      # base rows exactly zero
