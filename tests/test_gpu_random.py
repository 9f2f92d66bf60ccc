"""GPU parity on seeded random shapes: the dense SGEMM (NN and NT, with and
without bias) and the whole MoE layer (both routers, both activations, both
contraction modes, the planner's tile dealing and both forced ones), each
against the CPU oracle.  The shapes are drawn once from fixed seeds, so every
run checks the same cases; they reach the planner's tile shapes and K splits,
the skinny kernel, the register-staged fallback (K % 16 != 0, unaligned rows)
and ragged expert loads that the hand-picked cases leave out.

Bar: routing indices bit-exact, PHI weights bit-exact and softmax weights
within 1 ulp; activations within REL_TOL normwise relative error.
"""
import numpy as np
import pytest

from helpers import assert_close, load_pkg, normal

pytestmark = pytest.mark.gpu


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


def _sgemm_cases(n=48, seed=2024):
    rng = np.random.default_rng(seed)
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


def _layer_cases(n=48, seed=77):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        T = int(rng.integers(1, 900))
        d = int(rng.choice([int(rng.integers(1, 130)), 16 * int(rng.integers(1, 33))]))
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
