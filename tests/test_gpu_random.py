"""GPU parity on seeded random shapes: the dense SGEMM (NN and NT, with and
without bias), the whole MoE layer (both routers, both activations, both
contraction modes, the planner's tile dealing and both forced ones), the
router gate, causal attention and the two norms, each against the CPU oracle.  The shapes are drawn once from fixed seeds, so every
run checks the same cases; they reach the planner's tile shapes and K splits,
the skinny kernel, the register-staged fallback (K % 16 != 0, unaligned rows)
and ragged expert loads that the hand-picked cases leave out.

Bar: routing indices bit-exact, PHI weights bit-exact and softmax weights
within 1 ulp, gate logits and norms bit-exact; activations and attention within REL_TOL
normwise relative error.

MOE_RANDOM_CASES (default 48) sets how many cases each test draws (the
gate, attention and norm tests half as many) and MOE_RANDOM_SEED (default 0)
shifts the seeds, for a wider sweep by hand.
"""
import os

import numpy as np
import pytest

from helpers import assert_close, load_pkg, normal

pytestmark = pytest.mark.gpu

N_CASES = int(os.environ.get("MOE_RANDOM_CASES", "48"))
SEED = int(os.environ.get("MOE_RANDOM_SEED", "0"))


@pytest.fixture(scope="module")
def torch():
    import torch as _t
    assert _t.cuda.is_available(), "GPU tests need the MI355X"
    return _t


@pytest.fixture(scope="module")
def pkg():
    return load_pkg()


@pytest.fixture(scope="module")
def ctx(pkg, torch):
    c = pkg.Context(0)
    yield c
    c.close()


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def host(t):
    return t.detach().cpu().numpy()


def _sgemm_cases(n=N_CASES, seed=2024):
    rng = np.random.default_rng(seed + SEED)
    cases = []
    for i in range(n):
        M = int(rng.integers(1, 700))
        N = int(rng.integers(1, 800))
        K = int(rng.integers(0, 1500))
        if i % 3 == 0:
            K = 16 * max(1, K // 16)           # the direct-load kernels
        if i % 4 == 1:
            M = int(rng.integers(1, 33))         # the skinny kernel's rows
        if i % 5 == 2:
            N = 4 * max(1, N // 4)               # NN B rows of whole 16-byte chunks
        cases.append((M, N, K, bool(i % 2)))
    return cases


@pytest.mark.parametrize("M,N,K,with_bias", _sgemm_cases())
@pytest.mark.parametrize("layout", ["nn", "nt"])
def test_sgemm_random_shapes(ctx, torch, orc, layout, M, N, K, with_bias):
    print(f"sgemm {layout} {M}x{N}x{K} bias={with_bias}", flush=True)
    rng = np.random.default_rng(M * 7919 + N * 31 + K)
    a = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    b = rng.uniform(-1, 1, (K, N) if layout == "nn" else (N, K)).astype(np.float32)
    bias = rng.uniform(-1, 1, N).astype(np.float32) if with_bias else None
    c = torch.empty((M, N), device="cuda")
    fn = ctx.sgemm_nn if layout == "nn" else ctx.sgemm_nt
    fn(dev(torch, a), dev(torch, b), c, bias=None if bias is None else dev(torch, bias))
    ref = orc.matmul_nn(a, b) if layout == "nn" else orc.matmul_nt(a, b)
    if bias is not None:
        ref = ref + bias
    if K == 0:
        assert np.array_equal(host(c), ref)
    else:
        assert_close(host(c), ref, what=f"{layout} {M}x{N}x{K}")


def _layer_cases(n=N_CASES, seed=77):
    rng = np.random.default_rng(seed + SEED)
    cases = []
    while len(cases) < n:
        T = int(rng.integers(1, 900))
        d = int(rng.choice([int(rng.integers(1, 130)), 16 * int(rng.integers(1, 33))]))
        if rng.random() < 0.15:                  # wide rows, few tokens: split-K skinny w1/w3
            d, T = 1024 * int(rng.integers(1, 5)), int(rng.integers(1, 40))
        E = int(rng.integers(1, 80))
        k = int(rng.integers(1, min(E, 8) + 1))
        d_ff = int(rng.choice([int(rng.integers(1, 300)), 64 * int(rng.integers(1, 11))]))
        if T * k * d * d_ff * 3 > 4e8:           # keeps the oracle's share to seconds
            continue
        act = int(rng.integers(0, 2))
        router = int(rng.integers(0, 2))
        contract = int(rng.integers(0, 2))
        sk = int(rng.integers(-1, 2))
        cases.append((T, d, E, k, d_ff, act, router, contract, sk))
    return cases


@pytest.mark.parametrize("T,d,E,k,d_ff,act,router,contract,sk", _layer_cases())
def test_layer_random_shapes(ctx, pkg, torch, orc, T, d, E, k, d_ff, act, router, contract, sk):
    print(f"layer T={T} d={d} E={E} k={k} d_ff={d_ff} act={act} router={router} "
          f"contract={contract} sk={sk}", flush=True)
    ctx.set_stream_k(sk)
    try:
        rng = np.random.default_rng(T * 131 + d * 17 + E * 7 + d_ff)
        x = normal(rng, (T, d))
        gw = normal(rng, (E, d), 0.02)
        w1 = normal(rng, (E, d_ff, d), 0.02)
        w3 = normal(rng, (E, d_ff, d), 0.02) if act == 0 else None
        w2 = normal(rng, (E, d, d_ff), 0.02)
        desc = pkg.make_desc(T, d, E, k, d_ff, act=act, router=router, contract=contract)
        y = torch.empty((T, d), device="cuda")
        idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
        w = torch.empty((T, k), device="cuda")
        weights = {"gate_w": dev(torch, gw), "w1": dev(torch, w1),
                   "w3": None if w3 is None else dev(torch, w3), "w2": dev(torch, w2),
                   "expert_bias": None}
        ctx.layer_forward(desc, weights, dev(torch, x), y, idx, w)
        ry, ridx, rw = orc.moe_forward(x, gw, w1, w3, w2, k, act=act, router_mode=router,
                                       contract=contract)
        assert np.array_equal(host(idx), ridx), "routing"
        ulp = np.abs(host(w).view(np.int32).astype(np.int64) - rw.view(np.int32))
        assert ulp.max() <= (0 if router == 0 else 1), "routing weights"
        assert_close(host(y), ry, what="layer y")
    finally:
        ctx.set_stream_k(-1)


def _attention_cases(n=N_CASES // 2, seed=31):
    rng = np.random.default_rng(seed + SEED)
    cases = []
    while len(cases) < n:
        hd = int(rng.choice([64, 128, 64, 128, 16 * int(rng.integers(1, 9))]))
        fused = hd in (64, 128)
        S = int(rng.integers(1, 700)) if fused else 16 * int(rng.integers(1, 40))
        B = int(rng.integers(1, 5))
        KVH = int(rng.integers(1, 5))
        H = KVH * int(rng.integers(1, 5))
        window = int(rng.integers(1, S + 1)) if rng.random() < 0.4 else 0
        if B * H * S * S * hd > 2e8:             # keeps the oracle's share to seconds
            continue
        cases.append((B, S, H, KVH, hd, window))
    return cases


@pytest.mark.parametrize("B,S,H,KVH,hd,window", _attention_cases())
def test_attention_random_shapes(ctx, torch, orc, B, S, H, KVH, hd, window):
    """Causal attention (the fused kernel at head_dim 64 and 128, the batched
    GEMMs otherwise) on random batch, length, head and window shapes."""
    print(f"attention B={B} S={S} H={H} KVH={KVH} hd={hd} window={window}", flush=True)
    rng = np.random.default_rng(B * 1009 + S * 13 + H * 7 + KVH + hd + window)
    q = normal(rng, (B * S, H * hd))
    k = normal(rng, (B * S, KVH * hd))
    v = normal(rng, (B * S, KVH * hd))
    out = torch.full((B * S, H * hd), float("nan"), device="cuda")
    ctx.attention(dev(torch, q), dev(torch, k), dev(torch, v), out, B, S, H, KVH, hd, window)
    ref = orc.attention(q, k, v, B, S, H, KVH, hd, window or None)
    assert_close(host(out), ref, what="attention")


def _gate_cases(n=N_CASES // 2, seed=71):
    rng = np.random.default_rng(seed + SEED)
    cases = []
    for i in range(n):
        lo, hi = [(1, 8), (9, 16), (17, 80)][i % 3]
        E = int(rng.integers(lo, hi + 1))
        d = int(rng.integers(1, 4200))
        if i % 5 != 4:
            d = 4 * max(1, d // 4)               # 16-byte rows: the ring kernels
        few = 65536 // E                         # tokens of 65,536 logits
        T = int(rng.integers(1, few + 1)) if i % 2 == 0 else int(rng.integers(few + 1, 4 * few + 2))
        T = min(T, 40000)
        if T * d > 8_000_000:                    # x within 32 MB
            d = max(4, (8_000_000 // T) // 4 * 4)
        if T * E * d > 120_000_000:              # the oracle's chains, a second or so
            d = max(4, (120_000_000 // (T * E)) // 4 * 4)
        cases.append((T, d, E, (i // 2) % 2))
    return cases


@pytest.mark.parametrize("T,d,E,contract", _gate_cases())
def test_gate_random_shapes(ctx, torch, orc, T, d, E, contract):
    """The router gate on random shapes on both sides of every dispatch
    boundary (up to 8 experts: the per-wave ring; 9-64 with at most 65,536
    logits: the per-wave ring over expert blocks; 9-16 beyond: the workgroup
    ring; otherwise the staged kernel), rows aligned or not, bit for bit."""
    print(f"gate {T}x{d}x{E} contract={contract}", flush=True)
    rng = np.random.default_rng(T * 7 + d * 3 + E)
    x = normal(rng, (T, d))
    w = normal(rng, (E, d), 0.02)
    logits = torch.empty((T, E), device="cuda")
    ctx.gate_logits(dev(torch, x), dev(torch, w), logits, contract=contract)
    ref = orc.matmul_nt(x, w, contract=contract)
    assert np.array_equal(host(logits).view(np.int32), ref.view(np.int32))


def _norm_cases(n=N_CASES // 2, seed=53):
    rng = np.random.default_rng(seed + SEED)
    cases = []
    for i in range(n):
        rows = int(rng.integers(1, 3000))
        h = int(rng.integers(1, 6000))
        if i % 2 == 0:
            h = 4 * max(1, h // 4)               # 16-byte rows: the LDS and ring kernels
        if rows * h > 6_000_000:
            rows = max(1, 6_000_000 // h)
        cases.append((rows, h, bool(i % 3 == 0), i % 2))
    return cases


@pytest.mark.parametrize("rows,h,rms,contract", _norm_cases())
def test_norm_random_shapes(ctx, torch, orc, rows, h, rms, contract):
    """Layer norm and RMS norm on random row counts and widths (rows in LDS,
    the ring kernel, the register-staged pair), bit for bit."""
    print(f"{'rms' if rms else 'layer'}_norm {rows}x{h} contract={contract}", flush=True)
    rng = np.random.default_rng(rows * 5 + h * 3 + contract)
    x = (1 + 3 * rng.normal(size=(rows, h))).astype(np.float32)
    w = rng.normal(size=h).astype(np.float32)
    y = torch.empty((rows, h), device="cuda")
    inv = torch.empty(rows, device="cuda")
    if rms:
        ry, ri = orc.rms_norm(x, w, 1e-5, contract)
        ctx.rms_norm(dev(torch, x), dev(torch, w), y, 1e-5, contract, inv)
    else:
        b = rng.normal(size=h).astype(np.float32)
        ry, rm, ri = orc.layer_norm(x, w, b, 1e-5, contract)
        mean = torch.empty(rows, device="cuda")
        ctx.layer_norm(dev(torch, x), dev(torch, w), dev(torch, b), y, 1e-5, contract, mean, inv)
        assert np.array_equal(host(mean), rm), "mean"
    assert np.array_equal(host(inv), ri), "inv"
    assert np.array_equal(host(y), ry), "y"
