"""moe_layer_forward_noalloc (the layer on the library's fixed per-GPU
scratch, allocating nothing) against moe_layer_forward on the same inputs:
two calls in a row, the second with fewer tokens, each identical bit for bit
to the allocating entry point (the same kernels run on the same inputs);
and a layer too large for the scratch is rejected before any GPU work."""
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
            for noalloc in (False, True):
                y = torch.full((T, d), float("nan"), device="cuda")
                idx = torch.full((T, k), -1, dtype=torch.int32, device="cuda")
                w = torch.full((T, k), float("nan"), device="cuda")
                ctx.layer_forward(desc, W, x, y, idx, w, noalloc=noalloc)
                outs.append((y, idx, w))
            torch.cuda.synchronize()
            (y0, i0, w0), (y1, i1, w1) = outs
            assert torch.equal(i0, i1), f"T={T}: routing"
            assert torch.equal(w0, w1), f"T={T}: routing weights"
            assert torch.equal(y0, y1), f"T={T}: layer output"
            assert bool(torch.isfinite(y1).all())
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
