"""GPU parity of the decoder pieces around the MoE block (config 5's prefill):
RoPE, causal attention, the residual / bias adds and the embedding gather,
each through the C ABI against the CPU oracle on the same seeded inputs.

Bar: RoPE, the adds and the gather bit-exact (same table, same roundings);
attention within REL_TOL = 1e-4 normwise relative error (its two products
run on MFMA in another summation order than the oracle's serial loops).
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


# ------------------------------------------------------------------ RoPE
@pytest.mark.parametrize("B,S,H,KVH,hd,theta", [
    (1, 1, 1, 1, 2, 10000.0), (2, 9, 4, 2, 16, 10000.0), (3, 37, 3, 1, 6, 500000.0),
    (2, 100, 2, 0, 8, 10000.0), (8, 512, 16, 16, 64, 10000.0)])
def test_rope_bit_exact(ctx, torch, orc, B, S, H, KVH, hd, theta):
    print(f"rope B={B} S={S} H={H} KVH={KVH} hd={hd}", flush=True)
    rng = np.random.default_rng(B * 131 + S * 7 + hd)
    q = normal(rng, (B * S, H * hd))
    k = normal(rng, (B * S, max(KVH, 1) * hd))
    qd, kd = dev(torch, q), dev(torch, k)
    ctx.rope(qd, kd, B, S, H, KVH, hd, theta)
    rq, rk = orc.rope(q, k, B, S, H, KVH, hd, theta)
    assert np.array_equal(host(qd), rq)
    assert np.array_equal(host(kd), rk)


def test_rope_longer_table_and_errors(ctx, pkg, torch, orc):
    rng = np.random.default_rng(11)
    B, S, H, hd = 2, 12, 2, 8
    q, k = normal(rng, (B * S, H * hd)), normal(rng, (B * S, H * hd))
    qd, kd = dev(torch, q), dev(torch, k)
    table = ctx.rope_table(10000.0, hd, 64)  # rows past seq_len are never read
    ctx.rope(qd, kd, B, S, H, H, hd, table=table)
    rq, rk = orc.rope(q, k, B, S, H, H, hd)
    assert np.array_equal(host(qd), rq) and np.array_equal(host(kd), rk)
    short = ctx.rope_table(10000.0, hd, S - 1)
    with pytest.raises(pkg.MoeInvalidArgument):
        ctx.rope(qd, kd, B, S, H, H, hd, table=short)
    with pytest.raises(pkg.MoeInvalidArgument):
        ctx.rope(qd, kd, B, S, H, H, 7)


# ------------------------------------------------------------- attention
# (B, S, Hq, Hkv, hd, window): one tile; grouped query heads; a window inside
# one tile and across tiles; several 128-row tiles of a 64-wide head; a
# window of exactly S (unlimited); config 5's full prefill shape.
ATTN_CASES = [(1, 16, 1, 1, 16, None), (2, 48, 4, 2, 16, None), (2, 48, 4, 2, 16, 5),
              (1, 160, 2, 1, 64, None), (1, 160, 2, 1, 64, 130), (2, 272, 3, 3, 32, 20),
              (1, 144, 4, 1, 48, 144), (8, 512, 16, 16, 64, None)]


@pytest.mark.parametrize("B,S,H,KVH,hd,window", ATTN_CASES)
def test_attention_vs_oracle(ctx, torch, orc, B, S, H, KVH, hd, window):
    print(f"attention B={B} S={S} H={H} KVH={KVH} hd={hd} window={window}", flush=True)
    rng = np.random.default_rng(B * 17 + S + H * 5 + hd + (window or 0))
    q = normal(rng, (B * S, H * hd))
    k = normal(rng, (B * S, KVH * hd))
    v = normal(rng, (B * S, KVH * hd))
    out = torch.full((B * S, H * hd), float("nan"), device="cuda")
    ctx.attention(dev(torch, q), dev(torch, k), dev(torch, v), out, B, S, H, KVH, hd,
                  window or 0)
    ref = orc.attention(q, k, v, B, S, H, KVH, hd, window)
    assert_close(host(out), ref, what="attention")


def test_attention_after_rope_matches_the_oracle_chain(ctx, torch, orc):
    # the order the decoder runs them in: RoPE on q, k, then attention
    rng = np.random.default_rng(21)
    B, S, H, hd = 2, 64, 4, 32
    q, k, v = (normal(rng, (B * S, H * hd)) for _ in range(3))
    qd, kd = dev(torch, q), dev(torch, k)
    ctx.rope(qd, kd, B, S, H, H, hd)
    out = torch.empty((B * S, H * hd), device="cuda")
    ctx.attention(qd, kd, dev(torch, v), out, B, S, H, H, hd)
    rq, rk = orc.rope(q, k, B, S, H, H, hd)
    assert_close(host(out), orc.attention(rq, rk, v, B, S, H, H, hd), what="rope+attention")


def test_attention_unsupported_and_invalid_shapes(ctx, pkg, torch):
    z = torch.zeros(4096, device="cuda")
    with pytest.raises(pkg.MoeRuntimeError):  # seq_len not a multiple of 16
        ctx.attention(z, z, z, z, 1, 20, 2, 2, 16)
    with pytest.raises(pkg.MoeRuntimeError):  # head_dim not a multiple of 16
        ctx.attention(z, z, z, z, 1, 16, 2, 2, 8)
    with pytest.raises(pkg.MoeInvalidArgument):  # q heads not a multiple of kv heads
        ctx.attention(z, z, z, z, 1, 16, 3, 2, 16)
    with pytest.raises(pkg.MoeInvalidArgument):
        ctx.attention(z, z, z, z, 1, 16, 2, 2, 16, window=-1)
    ctx.attention(z, z, z, z, 0, 16, 2, 2, 16)  # no sequences: nothing to do


# ------------------------------------------------ adds and the embedding
@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 33), (4096, 1024)])
def test_add_and_add_bias_bit_exact(ctx, torch, rows, cols):
    rng = np.random.default_rng(rows + cols)
    a, b = normal(rng, (rows, cols)), normal(rng, (rows, cols))
    bias = normal(rng, (cols,))
    ad = dev(torch, a)
    ctx.add(ad, dev(torch, b))
    assert np.array_equal(host(ad), a + b)
    ctx.add_bias(ad, dev(torch, bias))
    assert np.array_equal(host(ad), (a + b) + bias[None, :])


def test_embed_gathers_rows_and_zeroes_out_of_range_tokens(ctx, torch):
    rng = np.random.default_rng(4)
    vocab, d, n = 1000, 96, 777
    table = normal(rng, (vocab, d))
    tokens = rng.integers(0, vocab, n).astype(np.int32)
    tokens[[3, 10]] = [-1, vocab]
    out = torch.full((n, d), float("nan"), device="cuda")
    ctx.embed(dev(torch, table), dev(torch, tokens), out)
    ref = table[np.clip(tokens, 0, vocab - 1)]
    ref[[3, 10]] = 0.0
    assert np.array_equal(host(out), ref)
