"""gather_qmm on the GPU against the oracle (the exact f64 contraction rounded
once). This is a floating-point contraction accumulated in f32, so the bar
is the stated tolerance, written here: every bf16/f16 output within 1 ulp of
the oracle, or within atol 1e-3 where the value sits next to zero (rtol 1e-2,
atol 1e-3); at least 99 % of outputs bit-identical."""
from __future__ import annotations

import numpy as np
import pytest

import higgs_amd as H
import oracle as O
from bits import assert_close, exact_frac
from gpu_util import to_dev, to_host, words_dev

pytestmark = pytest.mark.gpu


def _case(key, P, R, E, N, K, group=64, dt=O.BF16):
    x = O.from_f32(O.normal(key, (R, K)), dt)
    w = O.u32(key + 1, (E, N, K // 8))
    s = O.from_f32(O.uniform(key + 2, (E, N, K // group), 0.005, 0.02), dt)
    b = O.from_f32(O.uniform(key + 3, (E, N, K // group), -0.1, 0.1), dt)
    ex = (O.u32(key + 4, (P,)) % np.uint32(E)).astype(np.int32)
    return x, w, s, b, ex


def _run(dev, x, w, s, b, ex, dt, group=64, x_div=1, lhs=None):
    y = H.gather_qmm(to_dev(x, dt, dev), words_dev(w, dev), to_dev(s, dt, dev), to_dev(b, dt, dev),
                     to_dev(ex, O.I32, dev), group_size=group, x_row_div=x_div,
                     lhs_indices=None if lhs is None else to_dev(np.asarray(lhs, np.int32), O.I32, dev))
    return to_host(y)


def _check(got, ref, dt, what):
    ef = exact_frac(got, ref, dt)
    print(f"[qmm] {what}: exact={ef:.5f}", flush=True)
    assert_close(got, ref, dt, max_ulp=1, what=what)
    assert ef >= 0.99, what


@pytest.mark.parametrize("proj", ["gate_up", "down"])
def test_qwen3_next_decode_moe_shapes(dev, proj):
    """64 sequences x top-10 of 512 experts: gate/up (N 512, K 2048, x row =
    pair // 10) and down (N 2048, K 512, one activated row per pair)."""
    T, top_k, E = 64, 10, 512
    P = T * top_k
    if proj == "gate_up":
        x, w, s, b, ex = _case(2301, P, T, E, 512, 2048)
        x_div = top_k
    else:
        x, w, s, b, ex = _case(2311, P, P, E, 2048, 512)
        x_div = 1
    got = _run(dev, x, w, s, b, ex, O.BF16, x_div=x_div)
    ref = O.gather_qmm(x, O.BF16, w, s, b, O.BF16, ex, x_div=x_div)
    _check(got, ref, O.BF16, proj)


@pytest.mark.parametrize("N,group", [(300, 64), (1000, 32), (2112, 128)])
def test_short_rows_ragged_column_blocks(dev, N, group):
    """Short rows (K = 512, the down projection's shape class): row counts
    that leave the last 64-row block partly filled, each group size, and
    experts out of range."""
    P, R, E, K = 96, 96, 12, 512
    x, w, s, b, ex = _case(2380 + N + group, P, R, E, N, K, group=group)
    ex = ex.copy()
    ex[[3, 40]] = [E + 1, -2]  # out of range -> zero row; -2 wraps to E - 2
    got = _run(dev, x, w, s, b, ex, O.BF16, group=group)
    ref = O.gather_qmm(x, O.BF16, w, s, b, O.BF16, ex, group=group)
    _check(got, ref, O.BF16, f"N={N} g={group}")
    assert not got[3].any() and got[40].any()


@pytest.mark.parametrize("K,group", [(1024, 64), (4096, 64), (2048, 32), (2048, 128), (512, 32)])
def test_k_and_group_variants(dev, K, group):
    x, w, s, b, ex = _case(2320 + K + group, 37, 37, 9, 192, K, group=group)
    got = _run(dev, x, w, s, b, ex, O.BF16, group=group)
    ref = O.gather_qmm(x, O.BF16, w, s, b, O.BF16, ex, group=group)
    _check(got, ref, O.BF16, f"K={K} g={group}")


def test_f16_and_generic_shapes(dev):
    # f16 activations and scales, and a K that the vectorised kernel does not take
    for dt, K, N in ((O.F16, 2048, 256), (O.BF16, 192, 100), (O.BF16, 2048, 100)):
        x, w, s, b, ex = _case(2340 + K + N, 21, 7, 5, N, K)
        got = _run(dev, x, w, s, b, ex, dt, x_div=3)
        ref = O.gather_qmm(x, dt, w, s, b, dt, ex, x_div=3)
        _check(got, ref, dt, f"dt={dt} K={K} N={N}")


def test_routing_lhs_and_out_of_range(dev):
    P, R, E, N, K = 24, 5, 8, 128, 1024
    x, w, s, b, ex = _case(2361, P, R, E, N, K)
    lhs = (np.arange(P) * 7) % R
    ex = ex.copy()
    ex[[2, 9]] = [E + 3, -1]   # out of range -> zero row; -1 wraps to E - 1
    lhs[4] = R                 # row out of range -> zero row
    got = _run(dev, x, w, s, b, ex, O.BF16, lhs=lhs)
    ref = O.gather_qmm(x, O.BF16, w, s, b, O.BF16, ex, lhs=lhs)
    _check(got, ref, O.BF16, "lhs routing")
    assert not got[2].any() and not got[4].any() and got[9].any()


@pytest.mark.parametrize("K,x_div", [(512, 1), (1024, 3), (4096, 2)])
def test_decode_pairs_skewed_over_experts(dev, K, x_div):
    """Decode-sized pair counts (fewer than 16 per expert on average, so the
    per-pair kernel) with one expert holding 1500 of the 4000 pairs and the
    rest 0-8; a ragged N (200); an expert id out of range (zero row) and one
    that wraps (-1); K 512, 1024 and 4096 with x rows shared by 1-3 pairs."""
    P, E, N = 4000, 512, 200
    x, w, s, b, ex = _case(2440 + K, P, (P + x_div - 1) // x_div, E, N, K)
    ex = ex.copy()
    ex[100:1600] = 3
    ex[[5, 6]] = [E + 7, -1]
    got = _run(dev, x, w, s, b, ex, O.BF16, x_div=x_div)
    ref = O.gather_qmm(x, O.BF16, w, s, b, O.BF16, ex, x_div=x_div)
    _check(got, ref, O.BF16, f"skewed decode K={K}")
    assert not got[5].any() and got[6].any()


def test_swiglu_expert_block_end_to_end(dev):
    """forward_gather's whole expert block: gate and up gather_qmm, SwiGLU,
    down gather_qmm (qwen3_next.rs:868-904), against the oracle chain."""
    T, top_k, E, D, I = 16, 4, 32, 1024, 256
    P = T * top_k
    x = O.from_f32(O.normal(2371, (T, D)), O.BF16)
    ex = (O.u32(2372, (P,)) % np.uint32(E)).astype(np.int32)
    mats = {}
    for i, (nm, N, K) in enumerate((("gate", I, D), ("up", I, D), ("down", D, I))):
        mats[nm] = (O.u32(2380 + 4 * i, (E, N, K // 8)),
                    O.from_f32(O.uniform(2381 + 4 * i, (E, N, K // 64), 0.005, 0.02), O.BF16),
                    O.from_f32(O.uniform(2382 + 4 * i, (E, N, K // 64), -0.1, 0.1), O.BF16))
    g_ref = O.gather_qmm(x, O.BF16, *mats["gate"], O.BF16, ex, x_div=top_k)
    u_ref = O.gather_qmm(x, O.BF16, *mats["up"], O.BF16, ex, x_div=top_k)
    a_ref = O.glu(O.ACT_SILU, g_ref, u_ref, O.BF16)
    d_ref = O.gather_qmm(a_ref, O.BF16, *mats["down"], O.BF16, ex)

    tx = to_dev(x, O.BF16, dev)
    tex = to_dev(ex, O.I32, dev)
    dv = {k: (words_dev(w, dev), to_dev(s, O.BF16, dev), to_dev(b, O.BF16, dev)) for k, (w, s, b) in mats.items()}
    g = H.gather_qmm(tx, *dv["gate"], tex, x_row_div=top_k)
    u = H.gather_qmm(tx, *dv["up"], tex, x_row_div=top_k)
    _check(to_host(g), g_ref, O.BF16, "gate")
    act = H.swiglu(g, u)
    d = H.gather_qmm(act, *dv["down"], tex)
    # the down projection sees activations that may differ from the oracle's
    # in the last place (gate/up within 1 ulp), so compare it on the device's
    # own activations and check the chain end to end within the bar
    d_ref_dev = O.gather_qmm(to_host(act), O.BF16, *mats["down"], O.BF16, ex)
    _check(to_host(d), d_ref_dev, O.BF16, "down (device activations)")
    # three roundings deep, the end-to-end bar widens to 4 ulps
    assert_close(to_host(d), d_ref, O.BF16, max_ulp=4, what="expert block end to end")



def test_more_pairs_than_one_grid_holds(dev):
    """81,920 pairs exceed the 65535 pairs one launch of the per-pair kernel
    covers (6000 experts keep them below the grouped kernel's 16 pairs per
    expert); the pairs around the launch boundary and at both ends are
    checked against the oracle."""
    P, E, N, K = 81920, 6000, 16, 512
    x = O.from_f32(O.normal(2381, (P, K)), O.BF16)
    w = O.u32(2382, (E, N, K // 8))
    s = O.from_f32(O.uniform(2383, (E, N, K // 64), 0.005, 0.02), O.BF16)
    b = O.from_f32(O.uniform(2384, (E, N, K // 64), -0.1, 0.1), O.BF16)
    ex = (O.u32(2385, (P,)) % np.uint32(E)).astype(np.int32)
    got = _run(dev, x, w, s, b, ex, O.BF16)
    for lo, hi in ((0, 48), (65500, 65580), (P - 48, P)):
        ref = O.gather_qmm(x[lo:hi], O.BF16, w, s, b, O.BF16, ex[lo:hi])
        _check(got[lo:hi], ref, O.BF16, f"pairs {lo}..{hi}")


def test_grouped_prefill_path_matches_oracle(dev):
    """Many pairs per expert (a 512-token prefill at top-8 of 32 experts, 128
    pairs per expert on average) take the expert-grouped matrix-core kernel;
    gate/up style (x row = pair // top_k) and down style (one row per pair)."""
    T, top_k, E, N, K = 512, 8, 32, 256, 1024
    P = T * top_k
    w = O.u32(2401, (E, N, K // 8))
    s = O.from_f32(O.uniform(2402, (E, N, K // 64), 0.005, 0.02), O.BF16)
    b = O.from_f32(O.uniform(2403, (E, N, K // 64), -0.1, 0.1), O.BF16)
    ex = (O.u32(2404, (P,)) % np.uint32(E)).astype(np.int32)
    x = O.from_f32(O.normal(2405, (T, K)), O.BF16)
    got = _run(dev, x, w, s, b, ex, O.BF16, x_div=top_k)
    ref = O.gather_qmm(x, O.BF16, w, s, b, O.BF16, ex, x_div=top_k)
    _check(got, ref, O.BF16, "grouped gate/up")
    xd = O.from_f32(O.normal(2406, (P, K)), O.BF16)
    got = _run(dev, xd, w, s, b, ex, O.BF16)
    ref = O.gather_qmm(xd, O.BF16, w, s, b, O.BF16, ex)
    _check(got, ref, O.BF16, "grouped down")


@pytest.mark.parametrize("proj", ["gate_up", "down"])
def test_grouped_prefill_qwen3_next_shape(dev, proj):
    """The 4096-token Qwen3-Next MoE prefill bench.py times: top-10 of 512
    experts (40,960 pairs, ~80 per expert), gate/up 2048 -> 512 with x row =
    pair // 10, down 512 -> 2048 with one x row per pair. The whole call runs
    on the GPU; the oracle checks two blocks of 1024 pairs (every expert's
    list holds pairs from all over the call)."""
    T, top_k, E = 4096, 10, 512
    N, K = (512, 2048) if proj == "gate_up" else (2048, 512)
    P = T * top_k
    key = 2431 if proj == "gate_up" else 2441
    w = O.u32(key, (E, N, K // 8))
    s = O.from_f32(O.uniform(key + 1, (E, N, K // 64), 0.005, 0.02), O.BF16)
    b = O.from_f32(O.uniform(key + 2, (E, N, K // 64), -0.1, 0.1), O.BF16)
    ex = (O.u32(key + 3, (P,)) % np.uint32(E)).astype(np.int32)
    R, div = (T, top_k) if proj == "gate_up" else (P, 1)
    x = O.from_f32(O.normal(key + 4, (R, K)), O.BF16)
    got = _run(dev, x, w, s, b, ex, O.BF16, x_div=div)
    for lo in (0, P - 1024):
        sel = np.arange(lo, lo + 1024)
        ref = O.gather_qmm(x, O.BF16, w, s, b, O.BF16, ex[sel], lhs=(sel // div).astype(np.int32))
        _check(got[sel], ref, O.BF16, f"{proj} pairs {lo}..{lo + 1024}")
    # the order in which a block lists its expert's pairs depends on which
    # waves reach the list first; every row is computed on its own, so a
    # second call gives the same bits
    again = _run(dev, x, w, s, b, ex, O.BF16, x_div=div)
    assert np.array_equal(got, again), "a second call differs"


def test_grouped_hilo_path_for_other_k(dev):
    """Many pairs per expert with K not a multiple of 512 (9 groups): the
    grouped call runs the hi/lo-plane kernel instead of the exact-product
    one; gate/up style rows."""
    T, top_k, E, N, K = 384, 8, 16, 192, 576
    P = T * top_k
    w = O.u32(2451, (E, N, K // 8))
    s = O.from_f32(O.uniform(2452, (E, N, K // 64), 0.005, 0.02), O.BF16)
    b = O.from_f32(O.uniform(2453, (E, N, K // 64), -0.1, 0.1), O.BF16)
    ex = (O.u32(2454, (P,)) % np.uint32(E)).astype(np.int32)
    x = O.from_f32(O.normal(2455, (T, K)), O.BF16)
    got = _run(dev, x, w, s, b, ex, O.BF16, x_div=top_k)
    ref = O.gather_qmm(x, O.BF16, w, s, b, O.BF16, ex, x_div=top_k)
    _check(got, ref, O.BF16, "grouped hi/lo K=576")


def test_grouped_path_routing_and_out_of_range(dev):
    """The grouped kernel keeps gather_qmm's routing rules: lhs rows, -1
    wrapping to the last expert, out-of-range experts and rows giving zero
    rows; one expert with more pairs than one scan pass lists (the list is
    drained and the scan resumes)."""
    P, R, E, N, K = 10000, 40, 4, 128, 512
    x, w, s, b, ex = _case(2411, P, R, E, N, K)
    ex = ex.copy()
    ex[:9000] = 1                  # 9000 pairs on one expert: the list fills and drains
    ex[[5, 2300]] = [E + 2, -1]    # out of range -> zero row; -1 wraps to E - 1
    lhs = (np.arange(P) * 13) % R
    lhs[7] = R                     # row out of range -> zero row
    lhs[9] = -1                    # wraps to the last row
    got = _run(dev, x, w, s, b, ex, O.BF16, lhs=lhs)
    ref = O.gather_qmm(x, O.BF16, w, s, b, O.BF16, ex, lhs=lhs)
    _check(got, ref, O.BF16, "grouped routing")
    assert not got[5].any() and not got[7].any() and got[2300].any() and got[9].any()


@pytest.mark.parametrize("N", [200, 300])
def test_grouped_partial_column_tiles(dev, N):
    """The exact-product grouped kernel with a last column tile that is only
    partly inside the matrix: rows of 200 columns leave the tile through LDS
    as 16-byte pieces, rows of 300 (no multiple of 8) element by element."""
    P, R, E, K = 2048, 256, 4, 512
    x, w, s, b, ex = _case(2461 + N, P, R, E, N, K)
    got = _run(dev, x, w, s, b, ex, O.BF16, x_div=8)
    ref = O.gather_qmm(x, O.BF16, w, s, b, O.BF16, ex, x_div=8)
    _check(got, ref, O.BF16, f"grouped N={N}")


def test_grouped_size_with_unaligned_pair_count(dev):
    """A pair count that is not a multiple of 4 (the grouped kernel reads the
    expert ids 16 bytes at a time, so it leaves such a call to the per-pair
    kernel) gives the oracle's result, including the last pairs."""
    P, R, E, N, K = 4098, 600, 8, 128, 512
    x, w, s, b, ex = _case(2421, P, R, E, N, K)
    got = _run(dev, x, w, s, b, ex, O.BF16, x_div=7)
    ref = O.gather_qmm(x, O.BF16, w, s, b, O.BF16, ex, x_div=7)
    _check(got, ref, O.BF16, "unaligned pair count")
    _check(got[-2:], ref[-2:], O.BF16, "last pairs")


# ------------------------------------------------------------------ fused gate/up/SwiGLU
def _fused_case(key, T, top_k, E, N, K, group=64):
    P = T * top_k
    x = O.from_f32(O.normal(key, (T, K)), O.BF16)
    wg, wu = O.u32(key + 1, (E, N, K // 8)), O.u32(key + 2, (E, N, K // 8))
    sg = O.from_f32(O.uniform(key + 3, (E, N, K // group), 0.005, 0.02), O.BF16)
    bg = O.from_f32(O.uniform(key + 4, (E, N, K // group), -0.1, 0.1), O.BF16)
    su = O.from_f32(O.uniform(key + 5, (E, N, K // group), 0.005, 0.02), O.BF16)
    bu = O.from_f32(O.uniform(key + 6, (E, N, K // group), -0.1, 0.1), O.BF16)
    ex = (O.u32(key + 7, (P,)) % np.uint32(E)).astype(np.int32)
    return x, (wg, sg, bg), (wu, su, bu), ex


def _fused_dev(dev, x, g, u, ex, top_k, group=64):
    d = lambda t: to_dev(t, O.BF16, dev)
    return H.gather_qmm_swiglu(d(x), words_dev(g[0], dev), d(g[1]), d(g[2]), words_dev(u[0], dev),
                               d(u[1]), d(u[2]), to_dev(ex, O.I32, dev), group_size=group,
                               x_row_div=top_k)


@pytest.mark.parametrize("K,group", [(2048, 64), (512, 64), (1024, 32), (4096, 128)])
def test_fused_gate_up_swiglu_decode(dev, K, group):
    """64 sequences x top-10 of 512 experts (Qwen3-Next-80B-A3B's expert
    block at K 2048, N 512), and other K / group sizes. Bars: the one-launch
    form equals the reference's three calls run on the device bit for bit;
    it equals the oracle's SwiGLU applied to the device's two projections bit
    for bit; and those projections are within the contraction bar of the
    oracle's (1 ulp, 99 % exact). (The end result is not held to 1 ulp of the
    oracle's full composition: SiLU's relative slope 1 + g(1 - sigmoid(g))
    turns a 1-ulp difference in a gate value near g = -10 into ~9 ulp.)"""
    T, top_k, E, N = 64, 10, 512, 512
    x, g, u, ex = _fused_case(4000 + K + group, T, top_k, E, N, K, group)
    got = to_host(_fused_dev(dev, x, g, u, ex, top_k, group))
    d = lambda t: to_dev(t, O.BF16, dev)
    gd = H.gather_qmm(d(x), words_dev(g[0], dev), d(g[1]), d(g[2]), to_dev(ex, O.I32, dev),
                      group_size=group, x_row_div=top_k)
    ud = H.gather_qmm(d(x), words_dev(u[0], dev), d(u[1]), d(u[2]), to_dev(ex, O.I32, dev),
                      group_size=group, x_row_div=top_k)
    three = to_host(H.swiglu(gd, ud))
    assert np.array_equal(got, three), "fused result differs from gather_qmm, gather_qmm, swiglu"
    gh, uh = to_host(gd), to_host(ud)
    assert np.array_equal(got, O.glu(O.ACT_SILU, gh, uh, O.BF16)), "SwiGLU differs from the oracle's"
    rg = O.gather_qmm(x, O.BF16, g[0], g[1], g[2], O.BF16, ex, group=group, x_div=top_k)
    ru = O.gather_qmm(x, O.BF16, u[0], u[1], u[2], O.BF16, ex, group=group, x_div=top_k)
    _check(gh, rg, O.BF16, f"fused K={K} g={group}: gate projection")
    _check(uh, ru, O.BF16, f"fused K={K} g={group}: up projection")


def test_fused_gate_up_swiglu_grouped_prefill(dev):
    """The 4096-token Qwen3-Next MoE prefill (top-10 of 512 experts, 40,960
    pairs, N 512, K 2048) through the fused entry: the grouped matrix-core
    kernel's fused form. It equals the reference's three calls run on the
    device bit for bit, and the oracle's SwiGLU applied to the device's two
    projections; out-of-range experts give zero rows. With group 32 the fused
    grouped kernel does not apply and the Python form runs the three calls.
    Rows routed through lhs indices, one out of range, match the three calls
    too."""
    T, top_k, E, N, K = 4096, 10, 512, 512, 2048
    x, g, u, ex = _fused_case(4201, T, top_k, E, N, K)
    ex[[7, 20000]] = [E, -E - 1]
    got = to_host(_fused_dev(dev, x, g, u, ex, top_k))
    # same bits on a second call, whatever order the pairs are listed in
    assert np.array_equal(got, to_host(_fused_dev(dev, x, g, u, ex, top_k))), "a second call differs"
    d = lambda t: to_dev(t, O.BF16, dev)
    gh = to_host(H.gather_qmm(d(x), words_dev(g[0], dev), d(g[1]), d(g[2]), to_dev(ex, O.I32, dev),
                              x_row_div=top_k))
    uh = to_host(H.gather_qmm(d(x), words_dev(u[0], dev), d(u[1]), d(u[2]), to_dev(ex, O.I32, dev),
                              x_row_div=top_k))
    three = O.glu(O.ACT_SILU, gh, uh, O.BF16)
    assert np.array_equal(got, three), "fused grouped result differs from the three calls"
    assert not got[[7, 20000]].any()
    # the oracle on 2,560 pairs spread over the whole call (every 16th pair,
    # so every expert's list contributes): both projections within the
    # contraction bar, and the fused output equal to the oracle's SwiGLU of
    # the oracle's projections wherever the device's projections are the
    # oracle's (elsewhere SiLU's slope may widen a 1-ulp gate difference)
    rows = np.arange(0, T * top_k, 16)
    rows = rows[(rows != 7) & (rows != 20000)]
    rg = O.gather_qmm(x, O.BF16, g[0], g[1], g[2], O.BF16, ex[rows], lhs=rows // top_k)
    ru = O.gather_qmm(x, O.BF16, u[0], u[1], u[2], O.BF16, ex[rows], lhs=rows // top_k)
    _check(gh[rows], rg, O.BF16, "grouped fused: gate projection (sampled pairs)")
    _check(uh[rows], ru, O.BF16, "grouped fused: up projection (sampled pairs)")
    full = O.glu(O.ACT_SILU, rg, ru, O.BF16)
    same = (gh[rows] == rg) & (uh[rows] == ru)
    assert same.mean() >= 0.98, f"projections equal to the oracle's on {same.mean():.4f}"
    assert np.array_equal(got[rows][same], full[same]), "fused output differs from the oracle's SwiGLU"
    print(f"[qmm] grouped fused: output vs oracle composition exact={exact_frac(got[rows], full, O.BF16):.5f}",
          flush=True)
    # group 32: the fused grouped kernel does not take it
    T2, E2, K2 = 512, 8, 1024
    x2, g2, u2, ex2 = _fused_case(4211, T2, 4, E2, 256, K2, group=32)
    got2 = to_host(_fused_dev(dev, x2, g2, u2, ex2, 4, group=32))
    gh2 = to_host(H.gather_qmm(d(x2), words_dev(g2[0], dev), d(g2[1]), d(g2[2]),
                               to_dev(ex2, O.I32, dev), group_size=32, x_row_div=4))
    uh2 = to_host(H.gather_qmm(d(x2), words_dev(u2[0], dev), d(u2[1]), d(u2[2]),
                               to_dev(ex2, O.I32, dev), group_size=32, x_row_div=4))
    assert np.array_equal(got2, O.glu(O.ACT_SILU, gh2, uh2, O.BF16))
    # rows through lhs indices, one of them out of range (a zero row)
    T3, E3, N3, K3 = 512, 16, 256, 512
    P3 = T3 * 8
    x3, g3, u3, ex3 = _fused_case(4221, T3, 8, E3, N3, K3)
    lhs = ((np.arange(P3) * 37) % T3).astype(np.int32)
    lhs[11] = T3
    dl = to_dev(lhs, O.I32, dev)
    got3 = to_host(H.gather_qmm_swiglu(d(x3), words_dev(g3[0], dev), d(g3[1]), d(g3[2]),
                                       words_dev(u3[0], dev), d(u3[1]), d(u3[2]),
                                       to_dev(ex3, O.I32, dev), lhs_indices=dl))
    gh3 = to_host(H.gather_qmm(d(x3), words_dev(g3[0], dev), d(g3[1]), d(g3[2]),
                               to_dev(ex3, O.I32, dev), lhs_indices=dl))
    uh3 = to_host(H.gather_qmm(d(x3), words_dev(u3[0], dev), d(u3[1]), d(u3[2]),
                               to_dev(ex3, O.I32, dev), lhs_indices=dl))
    assert np.array_equal(got3, O.glu(O.ACT_SILU, gh3, uh3, O.BF16))
    assert not got3[11].any() and got3[12].any()
    # a partial last column tile written in 16-byte pieces (N 264) and rows
    # whose length is no multiple of 8 (N 300: written element by element)
    for N4 in (264, 300):
        x4, g4, u4, ex4 = _fused_case(4231 + N4, 512, 8, 16, N4, 512)
        got4 = to_host(_fused_dev(dev, x4, g4, u4, ex4, 8))
        gh4 = to_host(H.gather_qmm(d(x4), words_dev(g4[0], dev), d(g4[1]), d(g4[2]),
                                   to_dev(ex4, O.I32, dev), x_row_div=8))
        uh4 = to_host(H.gather_qmm(d(x4), words_dev(u4[0], dev), d(u4[1]), d(u4[2]),
                                   to_dev(ex4, O.I32, dev), x_row_div=8))
        assert np.array_equal(got4, O.glu(O.ACT_SILU, gh4, uh4, O.BF16)), f"N={N4}"


def test_fused_gate_up_swiglu_routing_and_fallback(dev):
    """Out-of-range experts give zero rows, as the three calls do; in the
    grouped (prefill) regime the fused entry runs the grouped kernel's fused
    form, here with many passes per expert (~1000 pairs each)."""
    T, top_k, E, N, K = 8, 4, 6, 256, 512
    x, g, u, ex = _fused_case(4101, T, top_k, E, N, K)
    ex[[1, 5, 9]] = [E, -E - 1, 1 << 20]
    got = to_host(_fused_dev(dev, x, g, u, ex, top_k))
    assert not got[[1, 5, 9]].any()
    keep = np.setdiff1d(np.arange(T * top_k), [1, 5, 9])
    d = lambda t: to_dev(t, O.BF16, dev)
    gh = to_host(H.gather_qmm(d(x), words_dev(g[0], dev), d(g[1]), d(g[2]), to_dev(ex, O.I32, dev),
                              x_row_div=top_k))
    uh = to_host(H.gather_qmm(d(x), words_dev(u[0], dev), d(u[1]), d(u[2]), to_dev(ex, O.I32, dev),
                              x_row_div=top_k))
    assert np.array_equal(got[keep], O.glu(O.ACT_SILU, gh, uh, O.BF16)[keep])
    # 2048 tokens x top-8 of 16 experts: ~1000 pairs per expert
    T2, E2 = 2048, 16
    x2, g2, u2, ex2 = _fused_case(4102, T2, 8, E2, 256, 512)
    got2 = to_host(_fused_dev(dev, x2, g2, u2, ex2, 8))
    rows = np.r_[0:64, T2 * 8 - 64:T2 * 8]
    d2 = lambda t: to_dev(t, O.BF16, dev)
    gh2 = to_host(H.gather_qmm(d2(x2), words_dev(g2[0], dev), d2(g2[1]), d2(g2[2]),
                               to_dev(ex2, O.I32, dev), x_row_div=8))
    uh2 = to_host(H.gather_qmm(d2(x2), words_dev(u2[0], dev), d2(u2[1]), d2(u2[2]),
                               to_dev(ex2, O.I32, dev), x_row_div=8))
    assert np.array_equal(got2, O.glu(O.ACT_SILU, gh2, uh2, O.BF16))
    rg2 = O.gather_qmm(x2, O.BF16, g2[0], g2[1], g2[2], O.BF16, ex2[rows], lhs=rows // 8)
    _check(gh2[rows], rg2, O.BF16, "grouped regime gate projection")
