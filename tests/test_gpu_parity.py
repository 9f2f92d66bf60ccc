"""GPU parity: every entry point of the C ABI against the CPU oracle on the
same seeded inputs.

Bar: routing indices, expert assignment, offsets, permutations and gate
logits bit-exact; activations within REL_TOL = 1e-4 normwise relative error
(helpers.REL_TOL); the combine is bit-exact given identical inputs.
"""
import ctypes
import json
import os

import numpy as np
import pytest

from helpers import (REL_TOL, assert_close, load_pkg, normal, rel_err, tile_cover_tokens,
                     zipf_bias)

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


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


@pytest.fixture
def request_reset_stream_k():
    """Calling it with a context puts that context back to the planner's
    stream-K choice when the test ends."""
    held = []
    yield held.append
    for c in held:
        c.set_stream_k(-1)


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def host(t):
    return t.detach().cpu().numpy()


# ------------------------------------------------------------------ SGEMM
# Besides edge shapes, these reach every dense tile shape and split-K path of
# the planner on a 256-CU MI355X: (40, 384, 4096) and (100, 300, 512) take the
# 32x128 tile with K splits, (64, 1408, 2048) the 64x128 tile with splits,
# (200, 520, 64) the 32x128 tile unsplit, (33, 250, 512) ragged M and N on a
# small tile, (64, 130, 256) an NN B whose rows are not 16-byte multiples.
# Up to 32 rows with K % 16 == 0 the skinny kernel runs: (1, 1000, 256) one
# row, (17, 200, 512) a second 16-row block 1 row deep and a last column block
# past N, (32, 132, 1024) two full row blocks with K splits, (9, 4, 64) one
# 4-column output; (5, 300, 48) and (20, 600, 1040) have K an odd multiple
# of 16, which admits no split.
SGEMM_SHAPES = [(1, 1, 1), (7, 5, 33), (129, 130, 17), (128, 128, 128),
                (256, 384, 512), (33, 200, 1000), (300, 64, 4), (5, 700, 2),
                (40, 384, 4096), (100, 300, 512), (64, 1408, 2048), (200, 520, 64),
                (33, 250, 512), (64, 130, 256), (1, 1000, 256), (17, 200, 512),
                (32, 132, 1024), (9, 4, 64), (5, 300, 48), (20, 600, 1040)]


@pytest.mark.parametrize("m,n,k", SGEMM_SHAPES)
def test_sgemm_nt_vs_oracle(ctx, torch, orc, m, n, k):
    print(f"sgemm_nt {m}x{n}x{k}", flush=True)
    rng = np.random.default_rng(m * 7 + n * 3 + k)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (n, k)).astype(np.float32)
    bias = rng.uniform(-1, 1, n).astype(np.float32)
    c = torch.empty((m, n), device="cuda")
    ctx.sgemm_nt(dev(torch, a), dev(torch, b), c)
    ref = orc.matmul_nt(a, b)
    assert_close(host(c), ref, what="nt")
    ctx.sgemm_nt(dev(torch, a), dev(torch, b), c, bias=dev(torch, bias))
    assert_close(host(c), ref + bias, what="nt+bias")


@pytest.mark.parametrize("m,n,k", SGEMM_SHAPES)
def test_sgemm_nn_vs_oracle(ctx, torch, orc, m, n, k):
    print(f"sgemm_nn {m}x{n}x{k}", flush=True)
    rng = np.random.default_rng(m * 5 + n * 11 + k)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    bias = rng.uniform(-1, 1, n).astype(np.float32)
    c = torch.empty((m, n), device="cuda")
    ctx.sgemm_nn(dev(torch, a), dev(torch, b), c)
    ref = orc.matmul_nn(a, b)
    assert_close(host(c), ref, what="nn")
    ctx.sgemm_nn(dev(torch, a), dev(torch, b), c, bias=dev(torch, bias))
    assert_close(host(c), ref + bias, what="nn+bias")


def test_sgemm_unaligned_k(ctx, torch, orc):
    # K % 4 != 0 takes the scalar-load path; a view at a 4-byte offset too
    rng = np.random.default_rng(9)
    a = rng.uniform(-1, 1, (70, 37)).astype(np.float32)
    b = rng.uniform(-1, 1, (90, 37)).astype(np.float32)
    c = torch.empty((70, 90), device="cuda")
    ctx.sgemm_nt(dev(torch, a), dev(torch, b), c)
    assert_close(host(c), orc.matmul_nt(a, b), what="K=37")
    big = torch.zeros(1 + 70 * 36, device="cuda")
    a2 = big[1:].view(70, 36)
    a2.copy_(dev(torch, a[:, :36]))
    ctx.sgemm_nt(a2, dev(torch, b[:, :36].copy()), c)
    assert_close(host(c), orc.matmul_nt(a[:, :36], b[:, :36]), what="offset A")


def test_sgemm_k_zero_gives_bias(ctx, torch):
    c = torch.full((3, 5), 7.0, device="cuda")
    bias = torch.arange(5, dtype=torch.float32, device="cuda")
    ctx.sgemm_nt(torch.empty((3, 0), device="cuda"), torch.empty((5, 0), device="cuda"),
                 c, bias=bias)
    assert np.array_equal(host(c), np.tile(np.arange(5, dtype=np.float32), (3, 1)))


@pytest.mark.parametrize("n", [1024, 2048])
def test_sgemm_square_config2(ctx, torch, orc, n):
    """Config-2 square shapes, fully checked against the oracle."""
    print(f"sgemm square {n}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(n)
    a = torch.rand((n, n), device="cuda", generator=g) * 2 - 1
    b = torch.rand((n, n), device="cuda", generator=g) * 2 - 1
    c = torch.empty((n, n), device="cuda")
    ctx.sgemm_nn(a, b, c)
    assert_close(host(c), orc.matmul_nn(host(a), host(b)), what=f"nn {n}")
    ctx.sgemm_nt(a, b, c)
    assert_close(host(c), orc.matmul_nt(host(a), host(b)), what=f"nt {n}")


@pytest.mark.parametrize("m,n,k", [(1000, 1000, 2048), (968, 1024, 512), (800, 1020, 768),
                                   (1024, 896, 1024)])
@pytest.mark.parametrize("layout", ["nn", "nt"])
def test_sgemm_k_groups(ctx, torch, orc, layout, m, n, k):
    """Shapes the planner deals to the K-group tile (32 x 128 tiles, one per
    CU for 3/4 to all of the CUs; four groups of 128-512 K columns each),
    with ragged row and column edges, with and without bias."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    tiles = -(-m // 32) * -(-n // 128)
    assert 4 * tiles >= 3 * cus and tiles <= cus and k % 64 == 0 and 128 <= k // 4 <= 512
    assert ctx.sgemm_plan(m, n, k, nn=layout == "nn") == {"tile": 5, "splits": 1}
    print(f"sgemm {layout} {m}x{n}x{k} (K groups)", flush=True)
    rng = np.random.default_rng(m * 3 + n * 5 + k)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (k, n) if layout == "nn" else (n, k)).astype(np.float32)
    bias = rng.uniform(-1, 1, n).astype(np.float32)
    c = torch.empty((m, n), device="cuda")
    fn = ctx.sgemm_nn if layout == "nn" else ctx.sgemm_nt
    ref = orc.matmul_nn(a, b) if layout == "nn" else orc.matmul_nt(a, b)
    fn(dev(torch, a), dev(torch, b), c)
    assert_close(host(c), ref, what=layout)
    fn(dev(torch, a), dev(torch, b), c, bias=dev(torch, bias))
    assert_close(host(c), ref + bias, what=layout + "+bias")


@pytest.mark.parametrize("m,n,k", [(16, 1000, 512), (48, 2048, 1024), (1024, 1024, 1024),
                                   (600, 700, 1000), (300, 257, 37), (2048, 4096, 512), (5, 7, 0)])
def test_sgemm_nt_residual(ctx, torch, orc, m, n, k):
    """moe_sgemm_nt_residual on shapes that reach the skinny kernel, split K,
    the K-group and 256-row tiles, the register-staged and scalar paths and
    K = 0: bit-identical to moe_sgemm_nt followed by the add (the residual is
    added after the bias in the store, or in the split reduction), within
    tolerance of the oracle, and in place (R == C)."""
    print(f"sgemm_nt_residual {m}x{n}x{k}", flush=True)
    rng = np.random.default_rng(m * 13 + n * 7 + k)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (n, k)).astype(np.float32)
    bias = rng.uniform(-1, 1, n).astype(np.float32)
    r = rng.uniform(-4, 4, (m, n)).astype(np.float32)
    da, db, dbias, dr = dev(torch, a), dev(torch, b), dev(torch, bias), dev(torch, r)
    plain = torch.empty((m, n), device="cuda")
    ctx.sgemm_nt(da, db, plain, bias=dbias)
    two_step = plain + dr
    fused = torch.empty((m, n), device="cuda")
    ctx.sgemm_nt(da, db, fused, bias=dbias, residual=dr)
    assert torch.equal(fused, two_step), "fused residual differs from GEMM + add"
    inplace = dr.clone()
    ctx.sgemm_nt(da, db, inplace, bias=dbias, residual=inplace)
    assert torch.equal(inplace, two_step), "in-place residual"
    ref = orc.matmul_nt(a, b) + bias + r
    if k == 0:
        assert np.array_equal(host(fused), (bias + r).astype(np.float32))
    else:
        assert_close(host(fused), ref, what="nt+bias+residual")


@pytest.mark.parametrize("n", [4096, 8192])
def test_sgemm_square_config2_row_sample(ctx, torch, orc, n):
    """Config-2 squares 4096^3 and 8192^3 through moe_sgemm_nn / moe_sgemm_nt
    (the planner's unsplit 128 x 128 tiles): the oracle recomputes whole
    output rows (each depends only on its A row), two in every 128-row m-tile
    at rotating positions, so every (m-tile, n-tile) output tile is checked."""
    print(f"sgemm square {n} (row sample)", flush=True)
    g = torch.Generator(device="cuda").manual_seed(n + 1)
    a = torch.rand((n, n), device="cuda", generator=g) * 2 - 1
    b = torch.rand((n, n), device="cuda", generator=g) * 2 - 1
    c = torch.empty((n, n), device="cuda")
    tiles = np.arange(n // 128)
    rows = np.unique(np.concatenate([tiles * 128 + (tiles * 37) % 128,
                                     tiles * 128 + 127 - (tiles * 11) % 64]))
    ah, bh = host(a[torch.from_numpy(rows).to("cuda")]), host(b)
    ctx.sgemm_nn(a, b, c)
    # the oracle's NN equals its NT on B^T bit for bit (tests/test_oracle.py);
    # the NT loop reads B row-wise, which a 256 MB B needs on the host
    assert_close(host(c[torch.from_numpy(rows).to("cuda")]),
                 orc.matmul_nt(ah, np.ascontiguousarray(bh.T)), what=f"nn {n} rows")
    ctx.sgemm_nt(a, b, c)
    assert_close(host(c[torch.from_numpy(rows).to("cuda")]), orc.matmul_nt(ah, bh),
                 what=f"nt {n} rows")


@pytest.mark.parametrize("m", [16, 64, 256, 512])
def test_sgemm_skinny_config2_row_sample(ctx, torch, orc, m):
    """Config-2 skinny expert shapes M x 14336 x 4096 at full size; the oracle
    recomputes a sample of rows (each output row depends only on its A row)."""
    print(f"sgemm skinny {m}", flush=True)
    n, k = 14336, 4096
    g = torch.Generator(device="cuda").manual_seed(m)
    a = torch.rand((m, k), device="cuda", generator=g) * 2 - 1
    b = torch.rand((k, n), device="cuda", generator=g) * 2 - 1
    c = torch.empty((m, n), device="cuda")
    ctx.sgemm_nn(a, b, c)
    rows = np.unique(np.linspace(0, m - 1, 8).astype(int))
    ref = orc.matmul_nn(host(a)[rows], host(b))
    assert_close(host(c)[rows], ref, what=f"skinny {m}")
    # split-K partials are summed in a fixed order: a second call is identical
    c2 = torch.empty_like(c)
    ctx.sgemm_nn(a, b, c2)
    assert torch.equal(c, c2)
    # the same product with B stored [N, K]
    bt = b.t().contiguous()
    del b
    ctx.sgemm_nt(a, bt, c2)
    assert_close(host(c2)[rows], ref, what=f"skinny nt {m}")


def test_sgemm_operands_past_2gib(ctx, torch, orc):
    """Operands whose per-tile byte offsets pass 2^31 take the kernel's 64-bit
    address path instead of the buffer loads: an NN B of 2 GiB and an NT B of
    128 rows of 2^22 floats, checked on a sample of outputs."""
    g = torch.Generator(device="cuda").manual_seed(31)
    print("sgemm nn 16 x 32768 x 16384 (B 2 GiB)", flush=True)
    m, n, k = 16, 32768, 16384
    a = torch.rand((m, k), device="cuda", generator=g) * 2 - 1
    b = torch.rand((k, n), device="cuda", generator=g) * 2 - 1
    c = torch.empty((m, n), device="cuda")
    ctx.sgemm_nn(a, b, c)
    cols = torch.tensor(np.linspace(0, n - 1, 64).astype(np.int64), device="cuda")
    ref = orc.matmul_nn(host(a), host(b[:, cols].contiguous()))
    assert_close(host(c[:, cols]), ref, what="nn past 2 GiB")
    del b, c
    print("sgemm nt 8 x 128 x 4194304 (B 2 GiB)", flush=True)
    m, n, k = 8, 128, 1 << 22
    a = torch.rand((m, k), device="cuda", generator=g) * 2 - 1
    b = torch.rand((n, k), device="cuda", generator=g) * 2 - 1
    c = torch.empty((m, n), device="cuda")
    ctx.sgemm_nt(a, b, c)
    rows, bn = [0, 7], [0, 1, 63, 64, 127]
    ref = orc.matmul_nt(host(a[rows]), host(b[bn]))
    assert_close(host(c[rows][:, bn]), ref, what="nt past 2 GiB")


# ------------------------------------------------------------ elementwise
def test_silu_mul_bit_exact(ctx, torch, orc):
    rng = np.random.default_rng(12)
    x = np.concatenate([np.linspace(-90, 90, 20001), rng.normal(size=5000) * 3,
                        [0.0, -0.0, 1e-30, -1e-30, 88.7, -88.7]]).astype(np.float32)
    u = normal(rng, x.shape)
    y = torch.empty(x.shape, device="cuda")
    ctx.silu(dev(torch, x), y)
    assert np.array_equal(host(y).view(np.int32), orc.silu(x).view(np.int32))
    p = torch.empty(x.shape, device="cuda")
    ctx.mul(y, dev(torch, u), p)
    assert np.array_equal(host(p), orc.mul(orc.silu(x), u))
    xt = dev(torch, x)
    ctx.silu(xt, xt)  # in place
    assert np.array_equal(host(xt).view(np.int32), orc.silu(x).view(np.int32))


# ------------------------------------------------------------------- gate
@pytest.mark.parametrize("contract", [0, 1])
# E <= 8 with 16-byte rows takes the ring kernel (64 x 512 x 4; 33 x 100 x 7:
# a partial last stage and a one-token last wave; 4096 x 1024 x 8, config
# 5's gate; 100 x 256 x 2: fewer experts than the lane block); E of 9-64 with
# 16-byte rows and at most 65,536 logits the same ring with 4-expert blocks
# over grid.y (300 x 4096 x 16 and 1037 x 4096 x 16: the reference's expert
# count, the latter with a partial last wave; 45 x 196 x 11: a partial last
# stage and expert block; 16 x 4 x 16: one 4-column stage; 1000 x 2048 x 64,
# config 4's expert count; 50 x 1024 x 32; 1 x 4096 x 16, one token); E of
# 9-16 with more logits the workgroup ring (4500 x 512 x 16, a partial last
# workgroup; 7000 x 260 x 10, 6 experts masked); every other shape the staged
# kernel: E above 64 (77 x 452 x 100: two 64-expert blocks, the second 36
# wide; grids of 512 workgroups or more, 4 tokens x 4 experts per thread:
# 33000 x 40 x 64 and 16421 x 96 x 100, ragged last workgroup and expert
# block) and rows that are not 16-byte multiples (70 x 130 x 130; 5 x 1 x 3)
@pytest.mark.parametrize("T,d,E", [(64, 512, 4), (300, 4096, 16), (1000, 2048, 64),
                                   (33, 100, 7), (5, 1, 3), (70, 130, 130), (4096, 1024, 8),
                                   (100, 256, 2), (1037, 4096, 16), (45, 196, 11),
                                   (77, 452, 100), (16, 4, 16), (50, 1024, 32),
                                   (33000, 40, 64), (16421, 96, 100), (1, 4096, 16),
                                   (4500, 512, 16), (7000, 260, 10)])
def test_gate_logits_bit_exact(ctx, torch, orc, contract, T, d, E):
    print(f"gate {T}x{d}x{E} contract={contract}", flush=True)
    rng = np.random.default_rng(T + d + E)
    x = normal(rng, (T, d))
    w = normal(rng, (E, d), 0.02)
    logits = torch.empty((T, E), device="cuda")
    ctx.gate_logits(dev(torch, x), dev(torch, w), logits, contract=contract)
    ref = orc.matmul_nt(x, w, contract=contract)
    assert np.array_equal(host(logits).view(np.int32), ref.view(np.int32))


@pytest.mark.parametrize("contract", [0, 1])
def test_routing_histogram_kat_on_gpu(ctx, torch, orc, contract):
    """The reference's published per-expert row counts
    (docs/microworld/exp-003-moe.html:399-405), recomputed by the GPU gate and
    router."""
    with open(os.path.join(GOLDEN, "exp003_routing_histogram.json")) as f:
        kat = json.load(f)
    gw = dev(torch, orc.lcg_fill((16, 4096), 101))
    for T_str, want in kat["rows_per_expert"].items():
        T = int(T_str)
        print(f"KAT T={T} contract={contract}", flush=True)
        x = dev(torch, orc.lcg_fill((T, 4096), 7 + T))
        logits = torch.empty((T, 16), device="cuda")
        ctx.gate_logits(x, gw, logits, contract=contract)
        idx = torch.empty((T, 2), dtype=torch.int32, device="cuda")
        w = torch.empty((T, 2), device="cuda")
        ctx.route(logits, 2, idx, w)
        got = np.bincount(host(idx).ravel(), minlength=16).tolist()
        assert got == want, f"T={T}"
        offsets = torch.empty(17, dtype=torch.int32, device="cuda")
        perm = torch.empty(2 * T, dtype=torch.int32, device="cuda")
        inv = torch.empty((T, 2), dtype=torch.int32, device="cuda")
        ctx.permute(idx, 16, offsets, perm, inv)
        assert np.diff(host(offsets)).tolist() == want


# ---------------------------------------------------------------- routing
@pytest.mark.parametrize("E,k", [(4, 2), (16, 2), (8, 2), (64, 8), (7, 3), (128, 4), (1, 1)])
@pytest.mark.parametrize("mode", [0, 1])
def test_route_vs_oracle(ctx, torch, orc, E, k, mode):
    print(f"route E={E} k={k} mode={mode}", flush=True)
    rng = np.random.default_rng(E * 10 + k + mode)
    T = 1000
    logits = normal(rng, (T, E), 0.1)
    logits[::5, :min(E, 3)] = logits[::5, :1]          # exact ties
    logits[1::9] = np.round(logits[1::9], 2)           # quantisation boundaries
    if E >= 3:
        logits[2::11, 2] = np.nan                      # NaN ranks as -inf (softmax)
    bias = zipf_bias(E) if E == 64 else None
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), device="cuda")
    ctx.route(dev(torch, logits), k, idx, w, mode=mode,
              expert_bias=None if bias is None else dev(torch, bias))
    ridx, rw = orc.route(logits, k, mode=mode, expert_bias=bias)
    assert np.array_equal(host(idx), ridx)
    if mode == 0:
        assert np.array_equal(host(w), rw)
    else:
        diff = np.abs(host(w).view(np.int32).astype(np.int64) - rw.view(np.int32))
        assert diff.max() <= 1, "softmax weights beyond 1 ulp"


def test_route_phi_hand_cases(ctx, torch, orc):
    rows = np.array([[0.0, 0.025, 0.04, -1.0], [0.5, 0.5, 0.5, 0.5],
                     [0.0, 0.0196, -1.0, -1.0], [0.0, 0.0194, -1.0, -1.0],
                     [-0.3, -0.2, -0.25, -0.9], [-0.0, 0.0, -1.0, -1.0]], np.float32)
    idx = torch.empty((6, 2), dtype=torch.int32, device="cuda")
    w = torch.empty((6, 2), device="cuda")
    ctx.route(dev(torch, rows), 2, idx, w)
    assert host(idx).tolist() == [[1, 2], [0, 1], [1, 0], [0, 1], [1, 2], [0, 1]]


# The layer routes and counts in one launch (route_count: each workgroup
# routes its tokens and adds its per-block expert counts into counters the
# gate launch zeroed), then places the pairs with the scan of those counts
# folded in (perm_place_scan; past kPlaceScanMax block counts, the separate
# scan and placement).  A layer of one permutation block (up to 256 tokens;
# for the softmax router at most two rounds of its lane groups) routes,
# scans and places in a single launch (route_place_one) instead.  Its
# routing, and through the outputs its offsets and permutation, against the
# oracle: one token, a partial block, exactly one block, a block plus one
# token, and 274 blocks; 1 to 1024 experts (softmax groups of 1 to 64 lanes,
# 4 to 256 tokens per round), k up to 32; the Zipf bias at E = 64; the
# one-block launch at 1, 16, 32, 100, 255 and 256 tokens with 1 to 1024
# experts.  Every case runs twice on the context: the second layer must find
# the counters, which the first left filled in the reused workspace, zeroed
# again by its own gate.
@pytest.mark.parametrize("T,E,k,mode", [(1, 4, 2, 1), (255, 8, 2, 1), (256, 16, 2, 0),
                                        (257, 64, 8, 1), (70000, 64, 8, 1), (70000, 16, 2, 0),
                                        (3001, 1, 1, 1), (1000, 100, 3, 0), (900, 1024, 32, 1),
                                        (600, 1024, 4, 0), (513, 3, 3, 1), (1, 1, 1, 0),
                                        (100, 1024, 32, 0), (32, 64, 8, 1), (16, 1024, 4, 1),
                                        (200, 5, 3, 0)])
def test_layer_fused_routing_vs_oracle(ctx, pkg, torch, orc, T, E, k, mode):
    print(f"layer routing T={T} E={E} k={k} mode={mode}", flush=True)
    rng = np.random.default_rng(T + 7 * E + k)
    d, d_ff = 64, 32
    x = normal(rng, (T, d))
    gw = normal(rng, (E, d), 0.3)
    w1 = normal(rng, (E, d_ff, d), 0.05)
    w3 = normal(rng, (E, d_ff, d), 0.05)
    w2 = normal(rng, (E, d, d_ff), 0.05)
    bias = zipf_bias(E) if E == 64 else None
    W = {"gate_w": dev(torch, gw), "w1": dev(torch, w1), "w3": dev(torch, w3),
         "w2": dev(torch, w2), "expert_bias": None if bias is None else dev(torch, bias)}
    desc = pkg.make_desc(T, d, E, k, d_ff, act=pkg.ACT_SWIGLU, router=mode)
    xt = dev(torch, x)
    outs = []
    for _ in range(2):
        y = torch.empty((T, d), device="cuda")
        idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
        w = torch.empty((T, k), device="cuda")
        ctx.layer_forward(desc, W, xt, y, idx, w)
        outs.append((host(y), host(idx), host(w)))
    ry, ridx, rw = orc.moe_forward(x, gw, w1, w3, w2, k, router_mode=mode, expert_bias=bias)
    for y, idx, w in outs:
        assert np.array_equal(idx, ridx)
        if mode == 0:
            assert np.array_equal(w, rw)
        else:
            diff = np.abs(w.view(np.int32).astype(np.int64) - rw.view(np.int32))
            assert diff.max() <= 1, "softmax weights beyond 1 ulp"
        assert_close(y, ry, what=f"T={T} E={E} k={k}")
    assert np.array_equal(outs[0][0], outs[1][0]), "second launch differs"


# ------------------------------------------------------------ permutation
def _rand_topk(rng, T, E, k, skew=False):
    if skew:
        p = np.arange(1, E + 1, dtype=np.float64) ** -1.2
        p /= p.sum()
        return np.stack([rng.choice(E, size=k, replace=False, p=p) for _ in range(T)]).astype(np.int32)
    return np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)


@pytest.mark.parametrize("T,E,k,skew", [(1, 4, 2, False), (255, 4, 2, False), (256, 8, 2, False),
                                        (1000, 64, 8, True), (3000, 16, 2, False),
                                        (777, 1024, 4, True), (513, 8, 8, False)])
def test_permute_bit_exact(ctx, torch, orc, T, E, k, skew):
    print(f"permute T={T} E={E} k={k}", flush=True)
    rng = np.random.default_rng(T + E + k)
    topk = _rand_topk(rng, T, E, k, skew)
    offsets = torch.empty(E + 1, dtype=torch.int32, device="cuda")
    perm = torch.empty(T * k, dtype=torch.int32, device="cuda")
    inv = torch.empty((T, k), dtype=torch.int32, device="cuda")
    ctx.permute(dev(torch, topk), E, offsets, perm, inv)
    roff, rperm, rinv = orc.permute(topk, E)
    assert np.array_equal(host(offsets), roff)
    assert np.array_equal(host(perm), rperm)
    assert np.array_equal(host(inv), rinv)


def test_permute_all_tokens_one_expert(ctx, torch, orc):
    T, E = 600, 8
    topk = np.stack([np.full(T, 5), np.full(T, 2)], axis=1).astype(np.int32)
    offsets = torch.empty(E + 1, dtype=torch.int32, device="cuda")
    perm = torch.empty(2 * T, dtype=torch.int32, device="cuda")
    inv = torch.empty((T, 2), dtype=torch.int32, device="cuda")
    ctx.permute(dev(torch, topk), E, offsets, perm, inv)
    roff, rperm, rinv = orc.permute(topk, E)
    assert np.array_equal(host(offsets), roff)
    assert np.array_equal(host(perm), rperm) and np.array_equal(host(inv), rinv)


# --------------------------------------------------------- FFN and combine
def _ffn_case(rng, T, d, E, k, d_ff, act, skew=False):
    x = normal(rng, (T, d))
    w1 = normal(rng, (E, d_ff, d), 0.02)
    w3 = normal(rng, (E, d_ff, d), 0.02) if act == 0 else None
    w2 = normal(rng, (E, d, d_ff), 0.02)
    topk = _rand_topk(rng, T, E, k, skew)
    return x, w1, w3, w2, topk


@pytest.mark.parametrize("T,d,E,k,d_ff,act,skew", [
    (64, 512, 4, 2, 1024, 1, False),     # config-1 expert shape, SiLU MLP
    (200, 256, 8, 2, 384, 0, False),
    (300, 128, 64, 8, 96, 0, True),      # ragged, tiny experts
    (50, 132, 4, 2, 70, 0, False),       # d, d_ff not multiples of the tile
    (33, 36, 16, 3, 17, 1, True),
    # d_ff % 128 == 64: w1/w3 on the 256 x 64 tile (dual SwiGLU, single SiLU,
    # and the register-staged kernel for K % 16 != 0)
    (700, 256, 8, 2, 448, 0, False),
    (150, 128, 4, 2, 192, 1, True),
    (90, 132, 4, 2, 320, 0, False),
    # more than 64 experts (the grouped kernels' expert lookup reads the
    # offsets instead of a register table); K = 32, two K steps per w1/w3 tile
    (400, 64, 100, 4, 64, 0, True),
    (100, 32, 8, 2, 64, 0, False),
])
@pytest.mark.parametrize("sk", [0, 1])
def test_expert_ffn_vs_oracle(ctx, torch, orc, request_reset_stream_k, T, d, E, k, d_ff, act,
                              skew, sk):
    """Both ways of dealing the grouped GEMMs' tiles: one tile per workgroup
    (sk 0) and stream-K with its fix-up of the cut tiles (sk 1; shapes whose
    K is not a multiple of 16 fall back to one tile per workgroup)."""
    print(f"ffn T={T} d={d} E={E} k={k} d_ff={d_ff} act={act} sk={sk}", flush=True)
    ctx.set_stream_k(sk)
    request_reset_stream_k(ctx)
    rng = np.random.default_rng(T + d + E + d_ff)
    x, w1, w3, w2, topk = _ffn_case(rng, T, d, E, k, d_ff, act, skew)
    roff, rperm, rinv = orc.permute(topk, E)
    ref = orc.expert_ffn(x, rperm, roff, w1, w3, w2, act=act)
    h = torch.empty((T * k, d_ff), device="cuda")
    out = torch.empty((T * k, d), device="cuda")
    ctx.expert_ffn_grouped(dev(torch, x), dev(torch, rperm), dev(torch, roff), dev(torch, w1),
                           None if w3 is None else dev(torch, w3), dev(torch, w2), k, h, out,
                           act=act)
    assert_close(host(out), ref, what="expert rows")


# Shapes the planner sends to the grouped skinny kernel (few rows per expert,
# K a multiple of 16; the context's default tile dealing): config 1's experts
# (32-row workgroups, SiLU), a decoder's last rows (8 tokens, 16-row
# workgroups, SwiGLU), every token on one expert (several row blocks for it,
# the others empty), and 16 experts with empty ones among them; w1/w3 split
# over K with the activation in the fix-up: the reference's experts at 8
# tokens (4 splits), SwiGLU at d 2048 (2), SiLU at d 2048 (2).  x misaligned
# by one float takes the tiles instead (same results within rounding).
@pytest.mark.parametrize("T,d,E,k,d_ff,act,route", [
    (64, 512, 4, 2, 1024, 1, "random"),
    (8, 1024, 8, 2, 2816, 0, "random"),
    (40, 256, 8, 2, 512, 0, "one"),
    (30, 128, 16, 4, 256, 1, "skew"),
    (5, 64, 4, 1, 64, 0, "random"),
    (8, 4096, 16, 2, 448, 0, "random"),
    (64, 2048, 8, 2, 512, 0, "random"),
    (16, 2048, 4, 1, 256, 1, "skew"),
])
@pytest.mark.parametrize("misaligned", [False, True])
def test_expert_ffn_skinny_vs_oracle(ctx, torch, orc, T, d, E, k, d_ff, act, route, misaligned):
    print(f"ffn skinny T={T} d={d} E={E} k={k} d_ff={d_ff} act={act} route={route} "
          f"misaligned={misaligned}", flush=True)
    rng = np.random.default_rng(T * 3 + d + E + d_ff)
    x, w1, w3, w2, topk = _ffn_case(rng, T, d, E, k, d_ff, act, route == "skew")
    if route == "one":
        topk = np.stack([np.roll(np.arange(E), -(t % 2))[:k] for t in range(T)]).astype(np.int32)
        topk[:, 0] = 0  # expert 0 takes every token
    roff, rperm, rinv = orc.permute(topk, E)
    ref = orc.expert_ffn(x, rperm, roff, w1, w3, w2, act=act)
    xd = dev(torch, x)
    if misaligned:
        buf = torch.empty(T * d + 1, device="cuda")
        buf[1:].copy_(xd.reshape(-1))
        xd = buf[1:].view(T, d)
    h = torch.empty((T * k, d_ff), device="cuda")
    out = torch.empty((T * k, d), device="cuda")
    ctx.expert_ffn_grouped(xd, dev(torch, rperm), dev(torch, roff), dev(torch, w1),
                           None if w3 is None else dev(torch, w3), dev(torch, w2), k, h, out,
                           act=act)
    assert_close(host(out), ref, what="expert rows")


@pytest.mark.parametrize("T,d,E,k,d_ff,act,splits", [(8, 1024, 8, 2, 2816, 0, 4),
                                                     (64, 512, 4, 2, 1024, 1, 4),
                                                     (24, 256, 16, 2, 448, 0, 1),
                                                     (8, 4096, 16, 2, 448, 0, 1)])
def test_layer_skinny_vs_oracle(ctx, pkg, torch, orc, T, d, E, k, d_ff, act, splits):
    """Whole layers on the grouped skinny kernel, w2 with the K splits the
    planner gives it (4 here for the first two, where the tiles would run w2
    unsplit under stream-K) summed by the combine: a decoder's last rows,
    config 1, the reference's experts at d 256 and at its d 4096 (w1/w3 split
    four ways over K)."""
    print(f"layer skinny T={T} d={d} E={E} k={k} d_ff={d_ff} act={act}", flush=True)
    rng = np.random.default_rng(T + d + E)
    x = normal(rng, (T, d))
    gw = normal(rng, (E, d), 0.02)
    w1 = normal(rng, (E, d_ff, d), 0.02)
    w3 = normal(rng, (E, d_ff, d), 0.02) if act == 0 else None
    w2 = normal(rng, (E, d, d_ff), 0.02)
    y, idx, w = _layer(ctx, pkg, torch, dev(torch, x), dev(torch, gw), dev(torch, w1),
                       None if w3 is None else dev(torch, w3), dev(torch, w2), k, act=act, mode=1)
    ry, ridx, rw = orc.moe_forward(x, gw, w1, w3, w2, k, act=act, router_mode=1)
    assert np.array_equal(host(idx), ridx)
    assert_close(host(y), ry, what="layer y")
    assert ctx.w2_splits(pkg.make_desc(T, d, E, k, d_ff, act=act, router=1)) == splits


def test_expert_ffn_gather_past_2gib(ctx, torch, orc):
    """x of 2 GiB: the w1/w3 row gather's byte offsets pass 2^31, so w1/w3 take
    the kernel's 64-bit address path (w2 reads packed rows from the tile's
    base and keeps the buffer loads).  Sampled tokens against the oracle run
    on just those tokens."""
    T, d, E, k, d_ff = 131072, 4096, 2, 1, 64
    print(f"ffn gather T={T} d={d} (x 2 GiB)", flush=True)
    g = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn((T, d), device="cuda", generator=g)
    rng = np.random.default_rng(7)
    w1, w3 = normal(rng, (E, d_ff, d), 0.02), normal(rng, (E, d_ff, d), 0.02)
    w2 = normal(rng, (E, d, d_ff), 0.02)
    topk = rng.integers(0, E, size=(T, k)).astype(np.int32)
    offsets = torch.empty(E + 1, dtype=torch.int32, device="cuda")
    perm = torch.empty(T * k, dtype=torch.int32, device="cuda")
    inv = torch.empty((T, k), dtype=torch.int32, device="cuda")
    ctx.permute(dev(torch, topk), E, offsets, perm, inv)
    h = torch.empty((T * k, d_ff), device="cuda")
    out = torch.empty((T * k, d), device="cuda")
    ctx.expert_ffn_grouped(x, perm, offsets, dev(torch, w1), dev(torch, w3), dev(torch, w2), k,
                           h, out)
    toks = np.unique(np.concatenate([[0, T - 1], rng.integers(0, T, size=62)]))
    sub_x = host(x[torch.from_numpy(toks).to("cuda")])
    roff, rperm, rinv = orc.permute(topk[toks], E)
    ref = orc.expert_ffn(sub_x, rperm, roff, w1, w3, w2, act=0)
    got = host(out[inv[torch.from_numpy(toks).to("cuda"), 0].long()])
    assert_close(got, ref[rinv[:, 0]], what="gathered rows past 2 GiB")


@pytest.mark.parametrize("contract", [0, 1])
# k = 2 (the two-slot path) with whole and partial column chunks, any other k
# in expert order, rows of d % 4 != 0 (scalar columns), k up to 32
@pytest.mark.parametrize("T,k,d", [(500, 8, 260), (300, 2, 4096), (129, 2, 1030), (77, 1, 64),
                                   (50, 32, 131), (40, 3, 4100), (3, 2, 1)])
def test_combine_bit_exact(ctx, torch, orc, contract, T, k, d):
    print(f"combine T={T} k={k} d={d} contract={contract}", flush=True)
    rng = np.random.default_rng(11 + T + k + d)
    topk = _rand_topk(rng, T, 64, k)
    roff, rperm, rinv = orc.permute(topk, 64)
    rows = normal(rng, (T * k, d))
    w = rng.uniform(0, 1, (T, k)).astype(np.float32)
    y = torch.empty((T, d), device="cuda")
    ctx.combine(dev(torch, rows), dev(torch, topk), dev(torch, w), dev(torch, rinv), y,
                contract=contract)
    ref = orc.combine(rows, topk, w, rinv, contract=contract)
    assert np.array_equal(host(y), ref)
    resid = normal(rng, (T, d))
    ctx.combine(dev(torch, rows), dev(torch, topk), dev(torch, w), dev(torch, rinv), y,
                resid=dev(torch, resid), contract=contract)
    assert np.array_equal(host(y), ref + resid)


# ------------------------------------------------------------ whole layer
def _layer(ctx, pkg, torch, x, gw, w1, w3, w2, k, act, mode, contract=1, bias=None):
    T, d = x.shape
    E, d_ff, _ = w1.shape
    desc = pkg.make_desc(T, d, E, k, d_ff, act=act, router=mode, contract=contract)
    y = torch.empty((T, d), device="cuda")
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), device="cuda")
    weights = {"gate_w": gw, "w1": w1, "w3": w3, "w2": w2, "expert_bias": bias}
    ctx.layer_forward(desc, weights, x, y, idx, w)
    return y, idx, w


def test_layer_config1(ctx, pkg, torch, orc):
    """Config 1: 64 tokens x 512, gate 512->4, top-2 softmax over the selected
    logits, SiLU-MLP experts 512->1024->512, weights N(0,0.02), x N(0,1), seed 0."""
    rng = np.random.default_rng(0)
    T, d, E, k, d_ff = 64, 512, 4, 2, 1024
    x = normal(rng, (T, d))
    gw = normal(rng, (E, d), 0.02)
    w1 = normal(rng, (E, d_ff, d), 0.02)
    w2 = normal(rng, (E, d, d_ff), 0.02)
    y, idx, w = _layer(ctx, pkg, torch, dev(torch, x), dev(torch, gw), dev(torch, w1), None,
                       dev(torch, w2), k, act=1, mode=1)
    ry, ridx, rw = orc.moe_forward(x, gw, w1, None, w2, k, act=1, router_mode=1)
    assert np.array_equal(host(idx), ridx)
    assert np.max(np.abs(host(w).view(np.int32).astype(np.int64) - rw.view(np.int32))) <= 1
    assert_close(host(y), ry, what="config1 y")


@pytest.mark.parametrize("contract,sk", [(0, -1), (1, -1), (1, 0), (1, 1)])
def test_layer_phi_router_swiglu(ctx, pkg, torch, orc, request_reset_stream_k, contract, sk):
    """The reference's own layer semantics: quantised top-2 with 0.5/0.5
    weights and SwiGLU experts (src/layer.cu:32-103), 16 experts; under the
    planner's tile dealing (sk -1) and both forced ones."""
    ctx.set_stream_k(sk)
    request_reset_stream_k(ctx)
    rng = np.random.default_rng(5)
    T, d, E, k, d_ff = 300, 256, 16, 2, 448
    x = normal(rng, (T, d))
    gw = normal(rng, (E, d), 0.02)
    w1 = normal(rng, (E, d_ff, d), 0.02)
    w3 = normal(rng, (E, d_ff, d), 0.02)
    w2 = normal(rng, (E, d, d_ff), 0.02)
    y, idx, w = _layer(ctx, pkg, torch, dev(torch, x), dev(torch, gw), dev(torch, w1),
                       dev(torch, w3), dev(torch, w2), k, act=0, mode=0, contract=contract)
    ry, ridx, rw = orc.moe_forward(x, gw, w1, w3, w2, k, act=0, router_mode=0,
                                   contract=contract)
    assert np.array_equal(host(idx), ridx) and np.array_equal(host(w), rw)
    assert_close(host(y), ry, what="phi layer y")


def test_layer_deterministic(ctx, pkg, torch):
    rng = np.random.default_rng(6)
    T, d, E, k, d_ff = 500, 128, 8, 2, 256
    args = [dev(torch, normal(rng, s, sd)) for s, sd in
            [((T, d), 1.0), ((E, d), 0.02), ((E, d_ff, d), 0.02), ((E, d_ff, d), 0.02),
             ((E, d, d_ff), 0.02)]]
    y1, i1, w1 = _layer(ctx, pkg, torch, *args, k, act=0, mode=1)
    y2, i2, w2 = _layer(ctx, pkg, torch, *args, k, act=0, mode=1)
    assert torch.equal(y1, y2) and torch.equal(i1, i2) and torch.equal(w1, w2)


def _check_all_routing(orc, xin, gw, k, mode, bias, idx, w, contract=1):
    """Routing of every token against the oracle's gate and router: indices
    bit-exact; weights bit-exact (PHI_QUANT) or within 1 ulp (softmax)."""
    logits = orc.matmul_nt(xin, gw, contract=contract)
    ridx, rw = orc.route(logits, k, mode=mode, expert_bias=bias)
    assert np.array_equal(idx, ridx), f"routing differs on {int(np.any(idx != ridx, axis=1).sum())} tokens"
    ulp = np.abs(w.view(np.int32).astype(np.int64) - rw.view(np.int32))
    assert ulp.max() <= (0 if mode == 0 else 1), "routing weights"


def _big_layer(ctx, pkg, torch, orc, T, d, E, k, d_ff, mode, bias, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn((T, d), device="cuda", generator=g)
    gw = torch.randn((E, d), device="cuda", generator=g) * 0.02
    w1 = torch.randn((E, d_ff, d), device="cuda", generator=g) * 0.02
    w3 = torch.randn((E, d_ff, d), device="cuda", generator=g) * 0.02
    w2 = torch.randn((E, d, d_ff), device="cuda", generator=g) * 0.02
    bias_t = None if bias is None else dev(torch, bias)
    y, idx, w = _layer(ctx, pkg, torch, x, gw, w1, w3, w2, k, act=0, mode=mode, bias=bias_t)
    gidx = host(idx)
    counts = np.bincount(gidx.ravel(), minlength=E)
    assert counts.sum() == T * k
    xh, gwh = host(x), host(gw)
    _check_all_routing(orc, xh, gwh, k, mode, bias, gidx, host(w))
    # every 128-row m-tile of every expert (both grouped GEMMs tile by 128
    # rows), its ragged last tile and the last token
    toks = tile_cover_tokens(gidx, E)
    print(f"full-size layer: routing of all {T} tokens bit-exact; oracle on {len(toks)} "
          f"tile-covering tokens", flush=True)
    ry, ridx, rw = orc.moe_forward(xh[toks], gwh, host(w1), host(w3), host(w2), k, act=0,
                                   router_mode=mode, expert_bias=bias)
    assert np.array_equal(gidx[toks], ridx)
    assert_close(host(y)[toks], ry, what="tile-covering tokens")
    return counts


def test_layer_mixtral_config3_full_size(ctx, pkg, torch, orc):
    """Config 3 at full size (4096 x 4096, E=8, top-2 softmax, SwiGLU 14336):
    routing of every token against the oracle, and the outputs of a token
    sample that covers every m-tile of every expert (routing is per token, so
    the oracle's layer on those tokens gives exactly their rows)."""
    counts = _big_layer(ctx, pkg, torch, orc, 4096, 4096, 8, 2, 14336, mode=1, bias=None,
                        seed=3)
    assert counts.min() > 0


def test_layer_skewed_config4_full_size(ctx, pkg, torch, orc):
    """Config 4 at full size (16384 x 2048, E=64, top-8, SwiGLU 1408, Zipf(1.2)
    router bias): routing of every token, outputs on a tile-covering sample."""
    counts = _big_layer(ctx, pkg, torch, orc, 16384, 2048, 64, 8, 1408, mode=1,
                        bias=zipf_bias(64), seed=4)
    assert counts.max() > 4 * counts.mean()  # heavily imbalanced loads


@pytest.mark.parametrize("T", [64, 1000])
def test_layer_reference_shape_small_batches(ctx, pkg, torch, orc, T):
    """The reference's layer shape at small batches, where the planner deals
    w1/w3 stream-K (64 tokens: a grid cut to keep pieces of 32 K steps;
    1000 tokens: every slot): routing of every token and the outputs of a
    tile-covering sample against the oracle."""
    ctx.set_stream_k(-1)
    _big_layer(ctx, pkg, torch, orc, T, 4096, 16, 2, 448, mode=0, bias=None, seed=60 + T)


def test_layer_reference_shape_full_size(ctx, pkg, torch, orc):
    """The reference's own layer shape (Phi-tiny-MoE: d 4096, 16 experts of
    d_ff 448, its quantised top-2 router) at its contest input's 15,583 rows:
    routing of every token, outputs on a tile-covering sample."""
    counts = _big_layer(ctx, pkg, torch, orc, 15583, 4096, 16, 2, 448, mode=0, bias=None,
                        seed=6)
    assert counts.min() > 0


# ------------------------------------------------------------- layer norm
@pytest.mark.parametrize("contract", [0, 1])
# rows held in LDS (whole rows per workgroup, 16-byte and scalar paths, h up
# to 1260 when aligned); wider aligned rows stream through the ring kernel with 8 or 32
# rows per wave (65 x 4096 and 3 x 30000: 8, a one-row last wave and a
# partial last stage; 8200 x 2600: 8 over many waves; 32800 x 2528: 32); 2 x 30001, wide
# and unaligned, takes the register-staged streaming pair
@pytest.mark.parametrize("rows,h", [(1, 1), (3, 5), (64, 64), (65, 4096), (200, 1000),
                                    (130, 33), (4096, 1024), (70, 20220), (3, 30000),
                                    (8200, 2600), (32800, 2528), (2, 30001)])
def test_layer_norm_bit_exact(ctx, torch, orc, contract, rows, h):
    print(f"layer_norm {rows}x{h} contract={contract}", flush=True)
    rng = np.random.default_rng(rows * 7 + h + contract)
    x = (2 + 3 * rng.normal(size=(rows, h))).astype(np.float32)
    w = rng.normal(size=h).astype(np.float32)
    b = rng.normal(size=h).astype(np.float32)
    ry, rm, ri = orc.layer_norm(x, w, b, 1e-5, contract)
    y = torch.empty((rows, h), device="cuda")
    mean = torch.empty(rows, device="cuda")
    inv = torch.empty(rows, device="cuda")
    ctx.layer_norm(dev(torch, x), dev(torch, w), dev(torch, b), y, 1e-5, contract, mean, inv)
    assert np.array_equal(host(mean), rm) and np.array_equal(host(inv), ri)
    assert np.array_equal(host(y), ry)
    # statistics only; and y alone (statistics in the workspace), in place
    mean.zero_()
    ctx.layer_norm(dev(torch, x), None, None, None, 1e-5, contract, mean, inv)
    assert np.array_equal(host(mean), rm)
    xd = dev(torch, x)
    ctx.layer_norm(xd, dev(torch, w), dev(torch, b), xd, 1e-5, contract)
    assert np.array_equal(host(xd), ry)


@pytest.mark.parametrize("contract", [0, 1])
@pytest.mark.parametrize("rows,h", [(1, 1), (3, 5), (65, 4096), (130, 33), (4096, 1024),
                                    (3, 30000), (8200, 2600), (2, 30001)])
def test_rms_norm_bit_exact(ctx, torch, orc, contract, rows, h):
    print(f"rms_norm {rows}x{h} contract={contract}", flush=True)
    rng = np.random.default_rng(rows * 3 + h + contract)
    x = (1 + 3 * rng.normal(size=(rows, h))).astype(np.float32)
    w = rng.normal(size=h).astype(np.float32)
    ry, ri = orc.rms_norm(x, w, 1e-5, contract)
    y = torch.empty((rows, h), device="cuda")
    inv = torch.empty(rows, device="cuda")
    ctx.rms_norm(dev(torch, x), dev(torch, w), y, 1e-5, contract, inv)
    assert np.array_equal(host(inv), ri) and np.array_equal(host(y), ry)
    xd = dev(torch, x)
    ctx.rms_norm(xd, dev(torch, w), xd, 1e-5, contract)  # in place, statistics in the workspace
    assert np.array_equal(host(xd), ry)


def _norm_block(ctx, pkg, torch, x, gw, w1, w3, w2, nw, nb, k, act, mode, contract,
                residual=True, bias=None, norm=None):
    T, d = x.shape
    E, d_ff, _ = w1.shape
    desc = pkg.make_desc(T, d, E, k, d_ff, act=act, router=mode, contract=contract,
                         norm=pkg.NORM_LAYER if norm is None else norm, norm_eps=1e-5,
                         residual=residual)
    y = torch.empty((T, d), device="cuda")
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), device="cuda")
    weights = {"gate_w": gw, "w1": w1, "w3": w3, "w2": w2, "expert_bias": bias,
               "norm_w": nw, "norm_b": nb}
    ctx.layer_forward(desc, weights, x, y, idx, w)
    return y, idx, w


def _norm_block_oracle(orc, x, gw, w1, w3, w2, nw, nb, k, act, mode, contract, residual,
                       bias=None, rms=False):
    if rms:
        xn, _ = orc.rms_norm(x, nw, 1e-5, contract)
    else:
        xn, _, _ = orc.layer_norm(x, nw, nb, 1e-5, contract)
    y, idx, w = orc.moe_forward(xn, gw, w1, w3, w2, k, act=act, router_mode=mode,
                                contract=contract, expert_bias=bias)
    return (y + x if residual else y), idx, w


# d = 256: 16-byte paths throughout; d = 198: scalar norm and GEMM loads
@pytest.mark.parametrize("d", [256, 198])
@pytest.mark.parametrize("mode,contract,act,rms", [(0, 0, 0, False), (0, 1, 0, False),
                                                   (1, 1, 0, False), (1, 0, 1, False),
                                                   (1, 1, 0, True), (0, 0, 1, True)])
def test_layer_norm_block_vs_oracle(ctx, pkg, torch, orc, d, mode, contract, act, rms):
    """The MoE block of the reference's decoder: y = x + MoE(layer_norm(x))
    (src/model.cu:1968-2021); routing bit-exact, y within the 1e-4 rule."""
    print(f"norm block d={d} mode={mode} contract={contract} act={act} rms={rms}", flush=True)
    rng = np.random.default_rng(d + 10 * mode + 100 * contract + act)
    T, E, k, d_ff = 300, 8, 2, 192
    x = (0.5 + 2 * rng.normal(size=(T, d))).astype(np.float32)
    gw = normal(rng, (E, d), 0.05)
    w1 = normal(rng, (E, d_ff, d), 0.05)
    w3 = normal(rng, (E, d_ff, d), 0.05) if act == 0 else None
    w2 = normal(rng, (E, d, d_ff), 0.05)
    nw = (1 + 0.1 * rng.normal(size=d)).astype(np.float32)
    nb = (0.1 * rng.normal(size=d)).astype(np.float32)
    y, idx, w = _norm_block(ctx, pkg, torch, dev(torch, x), dev(torch, gw), dev(torch, w1),
                            None if w3 is None else dev(torch, w3), dev(torch, w2),
                            dev(torch, nw), None if rms else dev(torch, nb), k, act, mode,
                            contract, norm=pkg.NORM_RMS if rms else pkg.NORM_LAYER)
    ry, ridx, rw = _norm_block_oracle(orc, x, gw, w1, w3, w2, nw, nb, k, act, mode, contract,
                                      residual=True, rms=rms)
    assert np.array_equal(host(idx), ridx)
    assert np.max(np.abs(host(w).view(np.int32).astype(np.int64) - rw.view(np.int32))) <= 1
    assert_close(host(y), ry, what="norm block y")


# The block at 9-16 experts (the reference's 16 and its workgroup-ring
# gate): one 64-column stage (d = 64), a partial last stage (d = 200, 1028),
# one token, a partial workgroup of tokens (T = 37), experts past E in the
# 16-expert block (E = 9, 12).
@pytest.mark.parametrize("T,d,E", [(1, 64, 16), (37, 200, 9), (1000, 1028, 12), (600, 4096, 16)])
@pytest.mark.parametrize("rms,contract", [(False, 1), (False, 0), (True, 1), (True, 0)])
def test_layer_norm_block_is_its_stages(ctx, pkg, torch, orc, T, d, E, rms, contract):
    """The block y = x + MoE(norm(x)) in one moe_layer_forward is
    bit-identical to its stages run apart: moe_layer_norm / moe_rms_norm,
    then the layer without a norm on the normalised rows, then + x; routing
    bit-exact against the oracle too."""
    print(f"norm block stages T={T} d={d} E={E} rms={rms} contract={contract}", flush=True)
    rng = np.random.default_rng(T + d + E + 7 * rms + 3 * contract)
    k, d_ff = 2, 96
    x = (0.5 + 2 * rng.normal(size=(T, d))).astype(np.float32)
    gw = normal(rng, (E, d), 0.05)
    w1 = normal(rng, (E, d_ff, d), 0.05)
    w3 = normal(rng, (E, d_ff, d), 0.05)
    w2 = normal(rng, (E, d, d_ff), 0.05)
    nw = (1 + 0.1 * rng.normal(size=d)).astype(np.float32)
    nb = (0.1 * rng.normal(size=d)).astype(np.float32)
    dx, dgw, dw1, dw3, dw2, dnw, dnb = (dev(torch, a) for a in (x, gw, w1, w3, w2, nw, nb))
    norm = pkg.NORM_RMS if rms else pkg.NORM_LAYER
    y, idx, w = _norm_block(ctx, pkg, torch, dx, dgw, dw1, dw3, dw2, dnw, None if rms else dnb,
                            k, pkg.ACT_SWIGLU, 0, contract, norm=norm)
    xn = torch.empty_like(dx)
    if rms:
        ctx.rms_norm(dx, dnw, xn, 1e-5, contract)
    else:
        ctx.layer_norm(dx, dnw, dnb, xn, 1e-5, contract)
    y0, idx0, w0 = _norm_block(ctx, pkg, torch, xn, dgw, dw1, dw3, dw2, None, None, k,
                               pkg.ACT_SWIGLU, 0, contract, residual=False, norm=pkg.NORM_NONE)
    assert torch.equal(idx, idx0) and torch.equal(w, w0)
    assert torch.equal(y, y0 + dx), "the block differs from its stages"
    _, ridx, _ = _norm_block_oracle(orc, x, gw, w1, w3, w2, nw, nb, k, 0, 0, contract,
                                    residual=True, rms=rms)
    assert np.array_equal(host(idx), ridx)


def test_layer_norm_block_without_residual(ctx, pkg, torch, orc):
    rng = np.random.default_rng(77)
    T, d, E, k, d_ff = 130, 128, 4, 2, 96
    x = normal(rng, (T, d))
    gw, w1, w3 = normal(rng, (E, d), 0.05), normal(rng, (E, d_ff, d), 0.05), normal(rng, (E, d_ff, d), 0.05)
    w2 = normal(rng, (E, d, d_ff), 0.05)
    nw, nb = normal(rng, (d,)), normal(rng, (d,), 0.1)
    y, idx, _ = _norm_block(ctx, pkg, torch, *[dev(torch, a) for a in (x, gw, w1, w3, w2, nw, nb)],
                            k, 0, 1, 1, residual=False)
    ry, ridx, _ = _norm_block_oracle(orc, x, gw, w1, w3, w2, nw, nb, k, 0, 1, 1, residual=False)
    assert np.array_equal(host(idx), ridx)
    assert_close(host(y), ry, what="norm block, no residual")


@pytest.mark.parametrize("norm", ["layer", "rms"])
def test_layer_norm_block_config5_moe_ffn(ctx, pkg, torch, orc, norm):
    """Config 5's MoE block at full size (8 x 512 tokens, d 1024, E=8, top-2,
    SwiGLU 2816) behind its norm (the RMSNorm config 5 names, and the
    reference's layer norm), with the residual: routing of every token against
    the oracle's norm, gate and router, and the block's output on a token
    sample covering every m-tile of every expert (every step is per token)."""
    print(f"config5 block norm={norm}", flush=True)
    rms = norm == "rms"
    T, d, E, k, d_ff = 4096, 1024, 8, 2, 2816
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn((T, d), device="cuda", generator=g) * 2 + 0.5
    gw = torch.randn((E, d), device="cuda", generator=g) * 0.02
    w1 = torch.randn((E, d_ff, d), device="cuda", generator=g) * 0.02
    w3 = torch.randn((E, d_ff, d), device="cuda", generator=g) * 0.02
    w2 = torch.randn((E, d, d_ff), device="cuda", generator=g) * 0.02
    nw = 1 + 0.1 * torch.randn(d, device="cuda", generator=g)
    nb = 0.1 * torch.randn(d, device="cuda", generator=g)
    y, idx, w = _norm_block(ctx, pkg, torch, x, gw, w1, w3, w2, nw, None if rms else nb, k, 0,
                            1, 1, norm=pkg.NORM_RMS if rms else pkg.NORM_LAYER)
    xh, gwh, nwh, nbh = host(x), host(gw), host(nw), host(nb)
    xn = orc.rms_norm(xh, nwh, 1e-5, 1)[0] if rms else orc.layer_norm(xh, nwh, nbh, 1e-5, 1)[0]
    gidx = host(idx)
    _check_all_routing(orc, xn, gwh, k, 1, None, gidx, host(w))
    toks = tile_cover_tokens(gidx, E)
    print(f"config5 block: routing of all {T} tokens bit-exact; oracle on {len(toks)} "
          f"tile-covering tokens", flush=True)
    ry, ridx, rw = _norm_block_oracle(orc, xh[toks], gwh, host(w1), host(w3), host(w2),
                                      nwh, nbh, k, 0, 1, 1, residual=True, rms=rms)
    assert np.array_equal(gidx[toks], ridx)
    assert_close(host(y)[toks], ry, what="config5 block, tile-covering tokens")


# ------------------------------------------------------------------ errors
def test_errors_are_reported(ctx, pkg, torch):
    c = torch.empty((4, 4), device="cuda")
    with pytest.raises(pkg.MoeInvalidArgument):
        ctx.sgemm_nt(torch.empty((4, 3), device="cuda"), torch.empty((4, 3), device="cuda"),
                     c.to(torch.float64))
    with pytest.raises(pkg.MoeInvalidArgument):
        ctx.route(torch.empty((4, 4), device="cuda"), 5,
                  torch.empty((4, 5), dtype=torch.int32, device="cuda"),
                  torch.empty((4, 5), device="cuda"))
    with pytest.raises(pkg.MoeInvalidArgument):
        pkg._check(pkg.load_library().moe_gate_logits(
            ctx.handle, None, None, None, 4, 8, 2000, 1, None))


def test_entry_points_reject_invalid_arguments(ctx, pkg, torch):
    """Every stage's argument checks, through the C ABI on a live context:
    null pointers at non-zero sizes, sizes out of range, unknown modes and a
    misaligned output each return MOE_ERR_INVALID with a message, before any
    launch; the context keeps working afterwards."""
    L = pkg.load_library()
    h = ctx.handle
    f = torch.zeros(64, device="cuda")
    i = torch.zeros(64, dtype=torch.int32, device="cuda")
    P, Q = f.data_ptr(), i.data_ptr()
    desc = pkg.make_desc(4, 8, 4, 2, 8, act=pkg.ACT_SWIGLU, router=0)
    wts = pkg.LayerWeights(P, None, P, P, P, None, None)
    bad_desc = pkg.make_desc(4, 8, 4, 2, 8, act=pkg.ACT_SWIGLU, router=0)
    bad_desc.residual = 2
    no_gate = pkg.LayerWeights(None, None, P, P, P, None, None)
    tile, splits = ctypes.c_int32(), ctypes.c_int32()
    cases = [
        ("silu", lambda: L.moe_silu(h, None, None, 16, None), "null pointer: x"),
        ("mul", lambda: L.moe_mul(h, P, P, P, -1, None), "n must be >= 0"),
        ("gate E=0", lambda: L.moe_gate_logits(h, P, P, P, 4, 8, 0, 1, None), "E must be in"),
        ("gate contract", lambda: L.moe_gate_logits(h, P, P, P, 4, 8, 4, 7, None), "contract"),
        ("route k>E", lambda: L.moe_route(h, P, None, 4, 4, 5, 0, 1e-3, 2e-2, Q, P, None),
         "k must be in"),
        ("route T", lambda: L.moe_route(h, P, None, 1 << 31, 4, 2, 0, 1e-3, 2e-2, Q, P, None),
         "T exceeds int32 range"),
        ("route mode", lambda: L.moe_route(h, P, None, 4, 4, 2, 9, 1e-3, 2e-2, Q, P, None),
         "router"),
        ("permute", lambda: L.moe_permute(h, Q, 4, 2, 4, None, Q, Q, None),
         "null pointer: expert_offsets"),
        ("ffn act", lambda: L.moe_expert_ffn_grouped(h, P, Q, Q, P, P, P, 7, 4, 2, 8, 8, 4, P,
                                                     P, None), "unknown act"),
        ("ffn w3", lambda: L.moe_expert_ffn_grouped(h, P, Q, Q, P, None, P, pkg.ACT_SWIGLU, 4, 2,
                                                    8, 8, 4, P, P, None), "null pointer: w3"),
        ("combine k", lambda: L.moe_combine(h, P, Q, P, Q, None, P, 4, 0, 8, 1, None),
         "k must be in"),
        ("combine misaligned y", lambda: L.moe_combine(h, P, Q, P, Q, None, P + 4, 4, 2, 8, 1,
                                                       None), "aligned"),
        ("layer residual", lambda: L.moe_layer_forward(h, ctypes.byref(bad_desc),
                                                       ctypes.byref(wts), P, P, None, None, None),
         "residual must be 0 or 1"),
        ("layer gate_w", lambda: L.moe_layer_forward(h, ctypes.byref(desc), ctypes.byref(no_gate),
                                                     P, P, None, None, None),
         "null pointer: gate_w"),
        ("attention heads", lambda: L.moe_attention(h, P, P, P, P, 1, 4, 4, 3, 8, 0, None),
         "heads"),
        ("rope head_dim", lambda: L.moe_rope(h, P, P, P, 8, 1, 4, 0, 1, 1, 3, None),
         "head_dim must be even"),
        ("layer_norm h", lambda: L.moe_layer_norm(h, P, P, P, 1e-5, 4, 0, 1, P, None, None, None),
         "h must be > 0"),
        ("sgemm M", lambda: L.moe_sgemm_nt(h, P, P, None, P, -1, 4, 4, None), "M must be >= 0"),
        ("sgemm N", lambda: L.moe_sgemm_nn(h, P, P, None, P, 4, 1 << 31, 4, None),
         "N exceeds int32 range"),
        ("stream-K mode", lambda: L.moe_ctx_set_stream_k(h, 2), "stream-K mode"),
        ("plan", lambda: L.moe_sgemm_plan(h, 1, 4, 4, 4, None, ctypes.byref(splits)),
         "null pointer: tile"),
        ("embed", lambda: L.moe_embed(h, P, Q, -1, 8, 8, P, None), "n must be >= 0"),
    ]
    for name, call, msg in cases:
        rc = call()
        err = L.moe_last_error().decode()
        assert rc == pkg.ERR_INVALID, (name, rc, err)
        assert msg in err, (name, err)
    torch.cuda.synchronize()
    # the context still works
    a = torch.arange(12, dtype=torch.float32, device="cuda").reshape(3, 4)
    c = torch.empty((3, 3), device="cuda")
    ctx.sgemm_nt(a, a, c)
    assert torch.equal(c.cpu(), a.cpu() @ a.cpu().T)
    assert L.moe_sgemm_plan(h, 1, 4, 4, 4, ctypes.byref(tile), ctypes.byref(splits)) == pkg.OK


@pytest.mark.parametrize("router", [0, 1])
def test_layer_empty_batch_and_single_expert(ctx, pkg, torch, orc, router):
    """T = 0: the call succeeds and writes nothing (the outputs keep their
    contents).  E = 1, k = 1: every token goes to the one expert; routing,
    weights and the layer output match the oracle."""
    print(f"layer edge cases router={router}", flush=True)
    d, d_ff = 64, 96
    rng = np.random.default_rng(11 + router)
    w = {"gate_w": dev(torch, normal(rng, (4, d), 0.1)),
         "w1": dev(torch, normal(rng, (4, d_ff, d), 0.05)),
         "w3": dev(torch, normal(rng, (4, d_ff, d), 0.05)),
         "w2": dev(torch, normal(rng, (4, d, d_ff), 0.05))}
    desc = pkg.make_desc(0, d, 4, 2, d_ff, act=pkg.ACT_SWIGLU, router=router)
    y0 = torch.full((1, d), 3.0, device="cuda")
    ctx.layer_forward(desc, w, torch.zeros((1, d), device="cuda"), y0)
    torch.cuda.synchronize()
    assert torch.all(y0 == 3.0)

    T = 37
    x = normal(rng, (T, d))
    gw = normal(rng, (1, d), 0.1)
    w1 = normal(rng, (1, d_ff, d), 0.05)
    w3 = normal(rng, (1, d_ff, d), 0.05)
    w2 = normal(rng, (1, d, d_ff), 0.05)
    desc = pkg.make_desc(T, d, 1, 1, d_ff, act=pkg.ACT_SWIGLU, router=router)
    y = torch.empty((T, d), device="cuda")
    idx = torch.full((T, 1), -1, dtype=torch.int32, device="cuda")
    tw = torch.empty((T, 1), device="cuda")
    ctx.layer_forward(desc, {"gate_w": dev(torch, gw), "w1": dev(torch, w1),
                             "w3": dev(torch, w3), "w2": dev(torch, w2)},
                      dev(torch, x), y, idx, tw)
    ry, ridx, rw = orc.moe_forward(x, gw, w1, w3, w2, 1, act=orc.ACT_SWIGLU,
                                   router_mode=router)
    assert np.array_equal(host(idx), ridx) and not np.any(host(idx))
    assert np.array_equal(host(tw), rw)
    assert_close(host(y), ry, what="E=1 layer")
