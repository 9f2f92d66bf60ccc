"""moe_layer_forward_noalloc (the layer on the library's fixed per-GPU
scratch, allocating nothing) against moe_layer_forward on the same inputs:
two calls in a row, the second with fewer tokens, each identical bit for bit
to the allocating entry point (the same kernels run on the same inputs),
on three chosen layers and 24 seeded random ones.  The no-alloc calls come first on a fresh context and must leave its
workspace at 0 bytes; one is captured in a HIP graph and replayed, with
other no-alloc calls between the replays, each replay matching the eager
call; and a layer too large for the scratch is rejected before any GPU
work."""
import numpy as np
import pytest

from helpers import load_pkg, normal

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as _t
    assert _t.cuda.is_available(), "GPU tests need the MI355X"
    return _t


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def _weights(torch, rng, d, E, d_ff, norm):
    w = {"gate_w": normal(rng, (E, d), 0.05), "w1": normal(rng, (E, d_ff, d), 0.05),
         "w3": normal(rng, (E, d_ff, d), 0.05), "w2": normal(rng, (E, d, d_ff), 0.05),
         "expert_bias": None}
    if norm:
        w["norm_w"] = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
        w["norm_b"] = normal(rng, (d,), 0.1)
    return {k: (None if v is None else _dev(torch, v)) for k, v in w.items()}


# (d, E, k, d_ff, router, norm, residual, T of the first call, T of the second):
# the reference's router and block (layer norm + residual) on 16 experts of
# d_ff 448, softmax top-4 on 64 experts with a K-split w2, and the reference's
# full width d 4096, whose w1/w3 runs stream-K (partial tiles in the scratch)
@pytest.mark.parametrize("d,E,k,d_ff,router,norm,residual,T1,T2", [
    (512, 16, 2, 448, 0, 1, True, 900, 333),
    (256, 64, 4, 96, 1, 0, False, 2000, 129),
    (4096, 16, 2, 448, 0, 0, False, 900, 333),
])
def test_noalloc_matches_layer_forward(torch, d, E, k, d_ff, router, norm, residual, T1, T2):
    pkg = load_pkg()
    print(f"noalloc d={d} E={E} k={k} d_ff={d_ff} T={T1} then {T2}", flush=True)
    rng = np.random.default_rng(d + E + T1)
    W = _weights(torch, rng, d, E, d_ff, norm)
    x_all = _dev(torch, normal(rng, (T1, d)))
    ctx = pkg.Context(0)
    try:
        for T in (T1, T2):
            desc = pkg.make_desc(T, d, E, k, d_ff, act=pkg.ACT_SWIGLU, router=router,
                                 norm=pkg.NORM_LAYER if norm else pkg.NORM_NONE,
                                 residual=residual)
            x = x_all[:T].contiguous()
            outs = []
            # the no-alloc call first: on this fresh context it must leave
            # the workspace unallocated (the allocating call then grows it)
            for noalloc in (True, False):
                y = torch.full((T, d), float("nan"), device="cuda")
                idx = torch.full((T, k), -1, dtype=torch.int32, device="cuda")
                w = torch.full((T, k), float("nan"), device="cuda")
                ws_before = ctx.workspace_bytes()
                ctx.layer_forward(desc, W, x, y, idx, w, noalloc=noalloc)
                if noalloc:
                    assert ctx.workspace_bytes() == ws_before, f"T={T}: no-alloc grew the workspace"
                    if T == T1:
                        assert ws_before == 0
                outs.append((y, idx, w))
            torch.cuda.synchronize()
            (y1, i1, w1), (y0, i0, w0) = outs
            assert torch.equal(i0, i1), f"T={T}: routing"
            assert torch.equal(w0, w1), f"T={T}: routing weights"
            assert torch.equal(y0, y1), f"T={T}: layer output"
            assert bool(torch.isfinite(y1).all())
    finally:
        ctx.close()


def _random_cases(n=24, seed=404):
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        d = int(rng.choice([int(rng.integers(1, 130)), 16 * int(rng.integers(1, 33))]))
        E = int(rng.integers(1, 80))
        k = int(rng.integers(1, min(E, 8) + 1))
        d_ff = int(rng.choice([int(rng.integers(1, 300)), 64 * int(rng.integers(1, 11))]))
        T1 = int(rng.integers(2, 1200))
        T2 = int(rng.integers(1, T1))
        cases.append((d, E, k, d_ff, int(rng.integers(0, 2)), int(rng.integers(0, 2)),
                      int(rng.integers(0, 3)), bool(rng.integers(0, 2)), T1, T2))
    return cases


# seeded random layers (odd widths, both activations and routers, no norm /
# layer norm / RMS norm, with and without the residual), each two no-alloc
# calls in a row against the allocating entry point, bit for bit
@pytest.mark.parametrize("d,E,k,d_ff,act,router,norm,residual,T1,T2", _random_cases())
def test_noalloc_random_shapes(torch, d, E, k, d_ff, act, router, norm, residual, T1, T2):
    pkg = load_pkg()
    print(f"noalloc random d={d} E={E} k={k} d_ff={d_ff} act={act} router={router} "
          f"norm={norm} residual={residual} T={T1} then {T2}", flush=True)
    rng = np.random.default_rng(d * 31 + E * 7 + T1)
    W = _weights(torch, rng, d, E, d_ff, norm != 0)
    if act != pkg.ACT_SWIGLU:
        W["w3"] = None
    x_all = _dev(torch, normal(rng, (T1, d)))
    norm_kind = [pkg.NORM_NONE, pkg.NORM_LAYER, pkg.NORM_RMS][norm]
    ctx = pkg.Context(0)
    try:
        for T in (T1, T2):
            desc = pkg.make_desc(T, d, E, k, d_ff, act=act, router=router, norm=norm_kind,
                                 residual=residual)
            x = x_all[:T].contiguous()
            outs = []
            for noalloc in (True, False):
                y = torch.full((T, d), float("nan"), device="cuda")
                idx = torch.full((T, k), -1, dtype=torch.int32, device="cuda")
                w = torch.full((T, k), float("nan"), device="cuda")
                ctx.layer_forward(desc, W, x, y, idx, w, noalloc=noalloc)
                outs.append((y, idx, w))
            torch.cuda.synchronize()
            (y1, i1, w1), (y0, i0, w0) = outs
            assert torch.equal(i0, i1), f"T={T}: routing"
            assert torch.equal(w0, w1), f"T={T}: routing weights"
            assert torch.equal(y0, y1), f"T={T}: layer output"
    finally:
        ctx.close()


def test_noalloc_replays_under_graph_capture(torch):
    # the reference's layer block (layer norm + residual, quantised top-2 of
    # 16 experts, d_ff 448) at d 512: one no-alloc call captured in a graph;
    # between its replays other no-alloc calls (other tokens, fewer of them)
    # overwrite the shared scratch, and every replay must still give the
    # eager call's result bit for bit
    pkg = load_pkg()
    d, E, k, d_ff, T, T2 = 512, 16, 2, 448, 700, 251
    print(f"noalloc graph d={d} E={E} T={T} (between replays T={T2})", flush=True)
    rng = np.random.default_rng(77)
    W = _weights(torch, rng, d, E, d_ff, True)
    x = _dev(torch, normal(rng, (T, d)))
    x2 = _dev(torch, normal(rng, (T2, d)))
    desc = pkg.make_desc(T, d, E, k, d_ff, act=pkg.ACT_SWIGLU, router=0, norm=pkg.NORM_LAYER,
                         residual=True)
    desc2 = pkg.make_desc(T2, d, E, k, d_ff, act=pkg.ACT_SWIGLU, router=0,
                          norm=pkg.NORM_LAYER, residual=True)
    ctx = pkg.Context(0)
    try:
        ref = torch.empty((T, d), device="cuda")
        ctx.layer_forward(desc, W, x, ref, noalloc=True)
        y = torch.empty((T, d), device="cuda")
        y2 = torch.empty((T2, d), device="cuda")
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            ctx.layer_forward(desc, W, x, y, noalloc=True)
        torch.cuda.synchronize()
        for rep in range(3):
            ctx.layer_forward(desc2, W, x2, y2, noalloc=True)
            y.fill_(float("nan"))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, ref), f"replay {rep} differs from the eager call"
        assert ctx.workspace_bytes() == 0
        del g
    finally:
        ctx.close()


def test_noalloc_rejects_a_layer_beyond_the_scratch(torch):
    pkg = load_pkg()
    ctx = pkg.Context(0)
    try:
        # config 3 at 4096 tokens needs about 600 MiB of workspace
        desc = pkg.make_desc(4096, 4096, 8, 2, 14336, act=pkg.ACT_SWIGLU,
                             router=pkg.ROUTER_SOFTMAX_TOPK)
        z = torch.zeros(16, device="cuda")
        W = {"gate_w": z, "w1": z, "w3": z, "w2": z}
        y = torch.full((16,), 3.0, device="cuda")
        with pytest.raises(pkg.MoeInvalidArgument, match="scratch"):
            ctx.layer_forward(desc, W, z, y, noalloc=True)
        torch.cuda.synchronize()
        assert bool((y == 3.0).all())
    finally:
        ctx.close()
