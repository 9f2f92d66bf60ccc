"""Pins the CPU oracle (oracle/moe_oracle.c) before anything is checked
against it.

Every check is chosen so that a plausible mistake fails it: the published
routing histograms of the reference (a known answer computed by the reference
itself), closed-form sums whose value depends on the summation order or on
the contraction, float64 brute force, and invariants.
"""
import json
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
F32 = np.float32


# ---------------------------------------------------------------- LCG + KAT
def test_lcg_first_values(orc):
    # s1 = 101*1664525 + 1013904223 mod 2^32; v = ((s1>>8)&0xFFFF)/32768 - 1
    s = 101
    vals = []
    for _ in range(3):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        vals.append(np.float32(((s >> 8) & 0xFFFF) / 32768.0 - 1.0))
    got = orc.lcg_fill((3,), 101)
    assert got.tolist() == vals


@pytest.mark.parametrize("contract", [0, 1])
def test_routing_histogram_matches_reference(orc, contract):
    """The reference's own per-expert row counts for its LCG-seeded MoE layer
    (docs/microworld/exp-003-moe.html:399-405) pin the LCG, the k-ascending
    gate GEMM and PhiMoE::route together, at six token counts."""
    with open(os.path.join(GOLDEN, "exp003_routing_histogram.json")) as f:
        kat = json.load(f)
    gw = orc.lcg_fill((16, 4096), 101)
    for T_str, want in kat["rows_per_expert"].items():
        T = int(T_str)
        x = orc.lcg_fill((T, 4096), 7 + T)
        logits = orc.matmul_nt(x, gw, contract=contract)
        idx, w = orc.route(logits, 2)
        assert np.all(w == F32(0.5))
        got = np.bincount(idx.ravel(), minlength=16).tolist()
        assert got == want, f"T={T}"
        assert np.all(idx[:, 0] != idx[:, 1])


# ------------------------------------------------------------------ SGEMM
def test_matmul_order_known_answer(orc):
    # [1e8, 1, -1e8, 1] . ones: k-ascending single accumulator gives
    # ((1e8+1)->1e8, -1e8 -> 0, +1) = 1; reversed gives 0, pairwise 0, exact 2.
    a = np.array([[1e8, 1.0, -1e8, 1.0]], dtype=F32)
    b = np.ones((1, 4), dtype=F32)
    for c in (0, 1):
        assert orc.matmul_nt(a, b, contract=c)[0, 0] == F32(1.0)
        assert orc.matmul_nn(a, b.T.copy(), contract=c)[0, 0] == F32(1.0)


def test_matmul_contraction_known_answer(orc):
    # acc = -(1+2^-11); then acc + (1+2^-12)^2.  The exact product is
    # 1 + 2^-11 + 2^-24: a fused multiply-add keeps the 2^-24, a separately
    # rounded product (ties-to-even) drops it.
    u = F32(1 + 2.0 ** -12)
    a = np.array([[F32(1 + 2.0 ** -11), u]], dtype=F32)
    b = np.array([[-1.0, u]], dtype=F32)
    assert orc.matmul_nt(a, b, contract=1)[0, 0] == F32(2.0 ** -24)
    assert orc.matmul_nt(a, b, contract=0)[0, 0] == F32(0.0)


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (7, 5, 33), (33, 17, 64), (64, 48, 257)])
def test_matmul_vs_float64(orc, m, n, k):
    rng = np.random.default_rng(m * 1000 + n * 10 + k)
    a = rng.uniform(-1, 1, (m, k)).astype(F32)
    b = rng.uniform(-1, 1, (n, k)).astype(F32)
    ref = a.astype(np.float64) @ b.astype(np.float64).T
    bound = k * 2.0 ** -23 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64).T) + 1e-30
    for c in (0, 1):
        got = orc.matmul_nt(a, b, contract=c)
        assert np.all(np.abs(got - ref) <= bound)
        # NN is the same loop nest over b read as [K, N]: bit-identical.
        assert np.array_equal(orc.matmul_nn(a, b.T.copy(), contract=c), got)


def test_matmul_empty(orc):
    c = orc.matmul_nt(np.zeros((0, 4), F32), np.zeros((3, 4), F32))
    assert c.shape == (0, 3)
    c = orc.matmul_nt(np.zeros((2, 0), F32), np.zeros((3, 0), F32))
    assert c.shape == (2, 3) and np.all(c == 0)


# ------------------------------------------------------------------- SiLU
def test_silu_properties(orc):
    x = np.linspace(-20, 20, 4001).astype(F32)
    y = orc.silu(x)
    assert orc.silu(np.zeros(1, F32))[0] == 0.0
    exact = x.astype(np.float64) / (1.0 + np.exp(-x.astype(np.float64)))
    # three roundings (exp to float, the add, the division): within 3 ulp
    ulp = np.spacing(np.abs(exact).astype(F32)).astype(np.float64)
    assert np.all(np.abs(y - exact) <= 3 * ulp + 1e-45)
    # silu(x) - silu(-x) = x
    assert np.allclose(y - orc.silu(-x), x, rtol=1e-6, atol=1e-6)


def test_mul(orc):
    a = np.array([1.5, -2.0, 3.0], F32)
    b = np.array([2.0, 0.25, -1.0], F32)
    assert orc.mul(a, b).tolist() == [3.0, -0.5, -3.0]


# ---------------------------------------------------------------- layer norm
@pytest.mark.parametrize("contract", [0, 1])
def test_layer_norm_closed_forms(orc, contract):
    eps = F32(1e-5)
    w = np.array([2.0, -3.0, 0.5, 4.0], F32)
    b = np.array([0.25, -1.0, 7.0, 0.0], F32)
    # a constant row: mean exact, var 0, inv = 1/sqrt(eps), y = bias exactly
    # (eps outside the sqrt, or a bias scaled by the weight, fail here)
    y, mean, inv = orc.layer_norm(np.full((1, 4), 3.0, F32), w, b, eps, contract)
    assert mean[0] == 3.0 and inv[0] == F32(1) / np.sqrt(eps)
    assert np.array_equal(y[0], b)
    # 1, 2, 3, 4: mean 2.5 and var 1.25 are exact in float
    x = np.array([[1, 2, 3, 4]], F32)
    y, mean, inv = orc.layer_norm(x, w, b, eps, contract)
    want_inv = F32(1) / np.sqrt(F32(1.25) + eps)
    assert mean[0] == 2.5 and inv[0] == want_inv
    scaled = (x[0] - F32(2.5)) * want_inv
    assert np.allclose(y[0], scaled * w + b, rtol=2e-7, atol=1e-7)


def test_layer_norm_single_float_accumulator(orc):
    # 1e8 absorbs each later 1 in a float accumulator, so the ascending float
    # sum is exactly 0; a double or compensated accumulator gives 16.
    row = np.array([[1e8] + [1.0] * 16 + [-1e8]], F32)
    one, zero = np.ones(18, F32), np.zeros(18, F32)
    _, mean, _ = orc.layer_norm(row, one, zero, 1e-5)
    assert mean[0] == 0.0


def test_layer_norm_two_pass_variance(orc):
    # mean 10002 is exact; the two-pass variance is (1 + 0 + 1) / 3.  The
    # one-pass E[x^2] - mean^2 loses it to cancellation (x^2 ~ 1e8).
    x = np.array([[10001.0, 10002.0, 10003.0]], F32)
    eps = F32(1e-5)
    _, mean, inv = orc.layer_norm(x, np.ones(3, F32), np.zeros(3, F32), eps)
    assert mean[0] == 10002.0
    assert inv[0] == F32(1) / np.sqrt(F32(2) / F32(3) + eps)


@pytest.mark.parametrize("contract", [0, 1])
def test_layer_norm_vs_float64(orc, contract):
    rng = np.random.default_rng(31 + contract)
    x = (3 + 2 * rng.normal(size=(20, 300))).astype(F32)
    w = rng.normal(size=300).astype(F32)
    b = rng.normal(size=300).astype(F32)
    y, mean, inv = orc.layer_norm(x, w, b, 1e-5, contract)
    x64 = x.astype(np.float64)
    m64 = x64.mean(axis=1)
    v64 = ((x64 - m64[:, None]) ** 2).mean(axis=1)
    i64 = 1 / np.sqrt(v64 + 1e-5)
    assert np.allclose(mean, m64, rtol=1e-5, atol=1e-6)
    assert np.allclose(inv, i64, rtol=1e-5)
    ref = (x64 - m64[:, None]) * i64[:, None] * w + b
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))


@pytest.mark.parametrize("contract", [0, 1])
def test_rms_norm_closed_forms(orc, contract):
    eps = F32(1e-5)
    w = np.array([2.0, -0.5, 3.0], F32)
    # constant row c: ss = 3 c^2 exactly (c = 2), inv = 1 / sqrt(c^2 + eps)
    y, inv = orc.rms_norm(np.full((1, 3), 2.0, F32), w, eps, contract)
    want_inv = F32(1) / np.sqrt(F32(4) + eps)
    assert inv[0] == want_inv
    assert np.array_equal(y[0], (F32(2) * want_inv) * w)
    # 3, 4: ss = 25, ss / 2 = 12.5 exact; a mean subtracted (layer norm's
    # slip) would give 0.25
    y, inv = orc.rms_norm(np.array([[3.0, 4.0]], F32), np.ones(2, F32), eps, contract)
    assert inv[0] == F32(1) / np.sqrt(F32(12.5) + eps)


def test_rms_norm_single_float_accumulator(orc):
    # 4096 squares of 1 after one 2^24: each 1 is absorbed in a float sum
    row = np.array([[4096.0] + [1.0] * 4096], F32)  # 4096^2 = 2^24
    _, inv = orc.rms_norm(row, np.ones(row.shape[1], F32), 0.0, 0)
    ss = F32(2 ** 24)  # the float chain: 2^24 + 1 rounds back to 2^24 every time
    assert inv[0] == F32(1) / np.sqrt(ss / F32(row.shape[1]))
    exact = F32(1) / np.sqrt(F32((2 ** 24 + 4096) / row.shape[1]))
    assert inv[0] != exact  # what a double accumulator would give


@pytest.mark.parametrize("contract", [0, 1])
def test_rms_norm_vs_float64(orc, contract):
    rng = np.random.default_rng(41 + contract)
    x = (1 + 2 * rng.normal(size=(17, 300))).astype(F32)
    w = rng.normal(size=300).astype(F32)
    y, inv = orc.rms_norm(x, w, 1e-5, contract)
    x64 = x.astype(np.float64)
    i64 = 1 / np.sqrt((x64 ** 2).mean(axis=1) + 1e-5)
    assert np.allclose(inv, i64, rtol=1e-5)
    ref = x64 * i64[:, None] * w
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))


# ---------------------------------------------------------------- RoPE
def test_rope_position_zero_is_identity_and_pairs_keep_length(orc):
    rng = np.random.default_rng(3)
    B, S, H, KVH, hd = 2, 9, 4, 2, 16
    q = rng.normal(size=(B * S, H * hd)).astype(F32)
    k = rng.normal(size=(B * S, KVH * hd)).astype(F32)
    rq, rk = orc.rope(q, k, B, S, H, KVH, hd)
    for b in range(B):  # position 0 of every sequence: cos 0 = 1, sin 0 = 0
        assert np.array_equal(rq[b * S], q[b * S]) and np.array_equal(rk[b * S], k[b * S])
    half = hd // 2
    for x, y in ((q, rq), (k, rk)):
        x3 = x.reshape(B * S, -1, hd).astype(np.float64)
        y3 = y.reshape(B * S, -1, hd).astype(np.float64)
        n0 = x3[..., :half] ** 2 + x3[..., half:] ** 2
        n1 = y3[..., :half] ** 2 + y3[..., half:] ** 2
        assert np.allclose(n0, n1, rtol=1e-5, atol=1e-6)


def test_rope_angles_vs_float64(orc):
    # one head, x = (1 on the first half, 0 on the second): pair j at position
    # s becomes (cos a, sin a) with a = s * theta^(-2j/hd)
    S, hd, theta = 40, 8, 10000.0
    q = np.zeros((S, hd), F32)
    q[:, : hd // 2] = 1.0
    rq, _ = orc.rope(q, q.copy(), 1, S, 1, 1, hd, theta)
    s = np.arange(S)[:, None].astype(np.float64)
    j = np.arange(hd // 2)[None, :].astype(np.float64)
    a = s * theta ** (-2 * j / hd)
    assert np.allclose(rq[:, : hd // 2], np.cos(a), atol=2e-6)
    assert np.allclose(rq[:, hd // 2:], np.sin(a), atol=2e-6)
    # the reference's frequency of pair j = hd/4: theta^(-1/2) = 0.01 at theta 1e4
    assert np.isclose(rq[1, hd // 4], np.cos(0.01), atol=1e-7)
    t = orc.rope_table(theta, hd, S)
    assert t.shape == (S, hd // 2, 2)
    assert np.allclose(t[..., 0], np.cos(a), atol=2e-6) and np.allclose(t[..., 1], np.sin(a),
                                                                        atol=2e-6)


def test_rope_quarter_turn_table_and_uncontracted_products(orc):
    rng = np.random.default_rng(5)
    S, H, hd = 3, 2, 8
    q = rng.normal(size=(S, H * hd)).astype(F32)
    k = rng.normal(size=(S, hd)).astype(F32)
    # cos 0 / sin 1 everywhere: (x0, x1) -> (-x1, x0) exactly
    t = np.zeros((S, hd // 2, 2), F32)
    t[..., 1] = 1.0
    rq, rk = orc.rope(q, k, 1, S, H, 1, hd, table=t)
    for x, y in ((q, rq), (k, rk)):
        x3, y3 = x.reshape(S, -1, hd), y.reshape(S, -1, hd)
        assert np.array_equal(y3[..., : hd // 2], -x3[..., hd // 2:])
        assert np.array_equal(y3[..., hd // 2:], x3[..., : hd // 2])
    # a generic table: each product rounds to float on its own (no FMA), the
    # rounding the reference's rope_rows spells out with __fmul_rn/__fsub_rn
    t = rng.uniform(-1, 1, (S, hd // 2, 2)).astype(F32)
    rq, _ = orc.rope(q, k, 1, S, H, 1, hd, table=t)
    q3 = q.reshape(S, H, hd)
    c, s = t[:, None, :, 0], t[:, None, :, 1]
    x0, x1 = q3[..., : hd // 2], q3[..., hd // 2:]
    exp0 = (x0 * c).astype(F32) - (x1 * s).astype(F32)
    exp1 = (x1 * c).astype(F32) + (x0 * s).astype(F32)
    assert np.array_equal(rq.reshape(S, H, hd), np.concatenate([exp0, exp1], axis=-1))
    fused = (x0.astype(np.float64) * c - (x1 * s).astype(F32)).astype(F32)
    assert not np.array_equal(fused, exp0)  # the inputs tell the two roundings apart


# ------------------------------------------------------------ attention
def test_attention_closed_forms(orc):
    rng = np.random.default_rng(8)
    B, S, H, KVH, hd = 2, 7, 4, 2, 8
    q = rng.normal(size=(B * S, H * hd)).astype(F32)
    k = rng.normal(size=(B * S, KVH * hd)).astype(F32)
    v = rng.normal(size=(B * S, KVH * hd)).astype(F32)
    out = orc.attention(q, k, v, B, S, H, KVH, hd)
    group = H // KVH
    for b in range(B):  # the first token of a sequence sees only itself: out = v
        for h in range(H):
            kh = h // group
            assert np.array_equal(out[b * S, h * hd:(h + 1) * hd], v[b * S, kh * hd:(kh + 1) * hd])
    # window 1: every token sees only itself
    out1 = orc.attention(q, k, v, B, S, H, KVH, hd, window=1)
    for h in range(H):
        kh = h // group
        assert np.array_equal(out1[:, h * hd:(h + 1) * hd], v[:, kh * hd:(kh + 1) * hd])
    # identical keys: uniform weights over the visible keys -> running mean of v
    kk = np.tile(k[:1], (B * S, 1))
    outu = orc.attention(q, kk, v, B, S, H, KVH, hd)
    for b in range(B):
        for qi in range(S):
            mean = v[b * S:b * S + qi + 1].astype(np.float64).mean(axis=0)
            assert np.allclose(outu[b * S + qi, :hd], mean[:hd], atol=1e-6)


@pytest.mark.parametrize("H,KVH,window", [(4, 4, None), (4, 2, None), (6, 3, 5)])
def test_attention_vs_float64(orc, H, KVH, window):
    rng = np.random.default_rng(H * 10 + KVH)
    B, S, hd = 2, 23, 16
    q = rng.normal(size=(B * S, H * hd)).astype(F32)
    k = rng.normal(size=(B * S, KVH * hd)).astype(F32)
    v = rng.normal(size=(B * S, KVH * hd)).astype(F32)
    out = orc.attention(q, k, v, B, S, H, KVH, hd, window=window)
    w = S if window is None else window
    ref = np.zeros_like(out, dtype=np.float64)
    for b in range(B):
        for h in range(H):
            kh = h // (H // KVH)
            Q = q[b * S:(b + 1) * S, h * hd:(h + 1) * hd].astype(np.float64)
            K = k[b * S:(b + 1) * S, kh * hd:(kh + 1) * hd].astype(np.float64)
            V = v[b * S:(b + 1) * S, kh * hd:(kh + 1) * hd].astype(np.float64)
            sc = Q @ K.T / np.sqrt(hd)
            i, j = np.indices((S, S))
            sc[(j > i) | (i - j >= w)] = -np.inf
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            ref[b * S:(b + 1) * S, h * hd:(h + 1) * hd] = p @ V
    assert np.max(np.abs(out - ref)) <= 1e-5 * np.max(np.abs(ref))


def test_layer_norm_contraction_differs(orc):
    # The FMA build fuses var += d*d and the weight/bias step; on random rows
    # that changes some outputs, and the unfused build is the float32 chain.
    rng = np.random.default_rng(5)
    x = rng.normal(size=(64, 257)).astype(F32)
    w = rng.normal(size=257).astype(F32)
    b = rng.normal(size=257).astype(F32)
    y1, _, _ = orc.layer_norm(x, w, b, 1e-5, 1)
    y0, m0, i0 = orc.layer_norm(x, w, b, 1e-5, 0)
    assert not np.array_equal(y0, y1)
    r = 3
    acc = F32(0)
    for v in x[r]:
        acc = F32(acc + v)
    mean = F32(acc / F32(257))
    var = F32(0)
    for v in x[r]:
        dv = F32(v - mean)
        var = F32(var + F32(dv * dv))
    inv = F32(F32(1) / np.sqrt(F32(var / F32(257)) + F32(1e-5)))
    assert m0[r] == mean and i0[r] == inv
    assert np.array_equal(y0[r], ((x[r] - mean) * inv) * w + b)


# ---------------------------------------------------------------- routing
def _phi(orc, row, k=2):
    idx, w = orc.route(np.array([row], F32), k)
    return tuple(idx[0].tolist())


def test_phi_route_hand_cases(orc):
    # Not an argmax: expert 1 beats 0 by > 0.02, expert 2 does not beat 1.
    assert _phi(orc, [0.0, 0.025, 0.04, -1.0]) == (1, 2)
    # Exact ties keep the lower index.
    assert _phi(orc, [0.5, 0.5, 0.5, 0.5]) == (0, 1)
    # 0.0196 quantises to 20 quanta, whose float value exceeds 0 + 0.02f.
    # An unquantised comparison would give (0, 1).
    assert _phi(orc, [0.0, 0.0196, -1.0, -1.0]) == (1, 0)
    # 0.0194 quantises to 19 quanta: not enough.
    assert _phi(orc, [0.0, 0.0194, -1.0, -1.0]) == (0, 1)
    # Signs are restored after quantising |s|.
    assert _phi(orc, [-0.3, -0.2, -0.25, -0.9]) == (1, 2)
    # -0 and +0 tie.
    assert _phi(orc, [-0.0, 0.0, -1.0, -1.0]) == (0, 1)
    # A quantum of 1e-3 makes 0.10004 and 0.1 equal.
    assert _phi(orc, [0.1, 0.10004, 0.13, 0.0]) == (2, 0)


def test_phi_route_weights(orc):
    rng = np.random.default_rng(0)
    idx, w = orc.route(rng.normal(size=(50, 16)).astype(F32), 2)
    assert np.all(w == F32(0.5))
    idx, w = orc.route(rng.normal(size=(50, 16)).astype(F32), 4)
    assert np.all(w == F32(0.25))
    assert all(len(set(r)) == 4 for r in idx.tolist())


def test_phi_route_bias_shifts_selection(orc):
    logits = np.zeros((3, 4), F32)
    bias = np.array([0.0, 0.0, 0.5, 0.3], F32)
    idx, _ = orc.route(logits, 2, expert_bias=bias)
    assert idx.tolist() == [[2, 3]] * 3


def test_softmax_topk_vs_brute_force(orc):
    rng = np.random.default_rng(1)
    for E, k in [(4, 2), (8, 2), (64, 8), (16, 16)]:
        logits = rng.normal(size=(200, E)).astype(F32)
        logits[::7, 1] = logits[::7, 0]  # exact ties
        bias = rng.normal(size=E).astype(F32) if E == 64 else None
        idx, w = orc.route(logits, k, mode=orc.ROUTER_SOFTMAX_TOPK,
                           expert_bias=bias)
        v = logits + (bias if bias is not None else 0)
        for t in range(v.shape[0]):
            order = sorted(range(E), key=lambda e: (-float(v[t, e]), e))[:k]
            assert idx[t].tolist() == order
            sel = v[t, order].astype(np.float64)
            ex = np.exp(sel - sel[0])
            ref = (ex / ex.sum()).astype(F32)
            assert np.all(np.abs(w[t].view(np.int32) - ref.view(np.int32)) <= 1)
        assert np.allclose(w.sum(axis=1), 1.0, atol=1e-6)


def test_softmax_topk_nan_ranks_last(orc):
    logits = np.array([[np.nan, 1.0, 2.0, np.nan]], F32)
    idx, w = orc.route(logits, 3, mode=orc.ROUTER_SOFTMAX_TOPK)
    assert idx[0].tolist() == [2, 1, 0]


def test_route_rejects_bad_k(orc):
    with pytest.raises(ValueError):
        orc.route(np.zeros((2, 4), F32), 5)
    with pytest.raises(ValueError):
        orc.route(np.zeros((2, 4), F32), 0)


# ------------------------------------------------------------ permutation
def test_permute_invariants_and_brute_force(orc):
    rng = np.random.default_rng(2)
    T, E, k = 300, 16, 4
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    offsets, perm, inv = orc.permute(idx, E)
    counts = np.bincount(idx.ravel(), minlength=E)
    assert offsets.tolist() == [0] + np.cumsum(counts).tolist()
    for e in range(E):
        want = [t for t in range(T) if e in idx[t]]
        assert perm[offsets[e]:offsets[e + 1]].tolist() == want
    for t in range(T):
        for s in range(k):
            r = inv[t, s]
            assert perm[r] == t and offsets[idx[t, s]] <= r < offsets[idx[t, s] + 1]


def test_permute_empty_experts_and_tokens(orc):
    idx = np.array([[3, 1], [3, 1]], np.int32)
    offsets, perm, inv = orc.permute(idx, 6)
    assert offsets.tolist() == [0, 0, 2, 2, 4, 4, 4]
    assert perm.tolist() == [0, 1, 0, 1]
    offsets, perm, inv = orc.permute(np.zeros((0, 2), np.int32), 4)
    assert offsets.tolist() == [0] * 5 and perm.size == 0


def test_permute_rejects_out_of_range(orc):
    with pytest.raises(ValueError):
        orc.permute(np.array([[0, 4]], np.int32), 4)


# ---------------------------------------------------------------- combine
def test_combine_ascending_expert_order(orc):
    # One token, experts listed as (2, 0, 1), unit weights; rows e0=1e8, e1=1,
    # e2=-1e8.  Ascending expert order: (1e8 + 1) -> 1e8, -1e8 -> 0.
    # Slot order would give (-1e8 + 1e8) + 1 = 1.
    out_rows = np.array([[-1e8], [1e8], [1.0]], F32)   # packed rows
    topk_idx = np.array([[2, 0, 1]], np.int32)
    inv = np.array([[0, 1, 2]], np.int32)
    w = np.ones((1, 3), F32)
    for c in (0, 1):
        assert orc.combine(out_rows, topk_idx, w, inv, contract=c)[0, 0] == 0.0


def test_combine_top2_closed_form(orc):
    rng = np.random.default_rng(3)
    rows = rng.normal(size=(8, 32)).astype(F32)
    topk_idx = np.array([[5, 1], [0, 7], [2, 3], [6, 4]], np.int32)
    inv = np.array([[0, 1], [2, 3], [4, 5], [6, 7]], np.int32)
    w = np.full((4, 2), 0.5, F32)
    y = orc.combine(rows, topk_idx, w, inv)
    want = F32(0.5) * rows[0::2] + F32(0.5) * rows[1::2]
    assert np.array_equal(y, want)


# ------------------------------------------------------- FFN and the layer
def _f64_layer(x, gw, w1, w3, w2, idx, w, act):
    x64 = x.astype(np.float64)
    T, d = x.shape
    y = np.zeros((T, d))
    for t in range(T):
        for s in range(idx.shape[1]):
            e = idx[t, s]
            g = w1[e].astype(np.float64) @ x64[t]
            h = g / (1 + np.exp(-g))
            if act == 0:
                h = h * (w3[e].astype(np.float64) @ x64[t])
            y[t] += float(w[t, s]) * (w2[e].astype(np.float64) @ h)
    return y


@pytest.mark.parametrize("act", [0, 1])
@pytest.mark.parametrize("mode", [0, 1])
def test_moe_forward_vs_float64(orc, act, mode):
    rng = np.random.default_rng(4 + act + 2 * mode)
    T, d, E, k, d_ff = 40, 64, 4, 2, 96
    x = rng.normal(size=(T, d)).astype(F32)
    gw = (0.02 * rng.normal(size=(E, d))).astype(F32)
    w1 = (0.02 * rng.normal(size=(E, d_ff, d))).astype(F32)
    w3 = (0.02 * rng.normal(size=(E, d_ff, d))).astype(F32)
    w2 = (0.02 * rng.normal(size=(E, d, d_ff))).astype(F32)
    y, idx, w = orc.moe_forward(x, gw, w1, w3 if act == 0 else None, w2, k,
                                act=act, router_mode=mode)
    ridx, rw = orc.route(orc.matmul_nt(x, gw), k, mode=mode)
    assert np.array_equal(idx, ridx) and np.array_equal(w, rw)
    ref = _f64_layer(x, gw, w1, w3, w2, idx, w, act)
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))


# ---------------------------------------------------- decoder composition
def _small_decoder(layers=2, seed=0):
    import torch
    from helpers import load_pkg
    pkg = load_pkg()
    cfg = pkg.DecoderConfig(layers=layers, d=32, heads=4, kv_heads=2, head_dim=8, experts=4,
                            top_k=2, d_ff=48, vocab=50)
    W = pkg.random_weights(cfg, "cpu", seed=seed)
    np_ = lambda t: None if t is None else t.numpy().copy()
    Wn = {k: np_(v) for k, v in W.items() if k != "layers"}
    Wn["layers"] = [{k: np_(v) for k, v in L.items()} for L in W["layers"]]
    return cfg, Wn


def test_decoder_layers_are_identities_when_their_weights_are_zero(orc):
    from oracle import decoder as od
    cfg, W = _small_decoder()
    for L in W["layers"]:
        for name in ("q_w", "k_w", "v_w", "o_w", "q_b", "k_b", "v_b", "o_b", "w1", "w3", "w2"):
            L[name][...] = 0.0
    tokens = np.random.default_rng(0).integers(0, cfg.vocab, (2, 5))
    logits, x, _ = od.generate(tokens, W, cfg)
    assert np.array_equal(x, W["embed"][tokens.reshape(-1)])
    last = W["embed"][tokens[:, -1]]
    ref = od.linear(od.norm(last, W["final_norm_w"], W["final_norm_b"], cfg), W["lm_head_w"],
                    W["lm_head_b"], cfg.contract)
    assert np.array_equal(logits, ref)
    # only o_proj's bias left: every layer adds it once to every row
    for L in W["layers"]:
        L["o_b"][...] = 0.25
    _, x2, _ = od.generate(tokens, W, cfg)
    assert np.allclose(x2, W["embed"][tokens.reshape(-1)] + 0.25 * cfg.layers, atol=1e-6)


def test_decoder_is_causal_and_sequences_are_independent(orc):
    from oracle import decoder as od
    cfg, W = _small_decoder()
    rng = np.random.default_rng(1)
    B, S = 3, 7
    tokens = rng.integers(0, cfg.vocab, (B, S))
    _, x, _ = od.generate(tokens, W, cfg)
    t2 = tokens.copy()
    t2[1, 4] = (t2[1, 4] + 1) % cfg.vocab  # sequence 1, position 4
    _, x2, _ = od.generate(t2, W, cfg)
    x3, x23 = x.reshape(B, S, -1), x2.reshape(B, S, -1)
    assert np.array_equal(x3[[0, 2]], x23[[0, 2]])       # other sequences untouched
    assert np.array_equal(x3[1, :4], x23[1, :4])         # earlier positions untouched
    assert not np.array_equal(x3[1, 4:], x23[1, 4:])     # the rest sees the change
