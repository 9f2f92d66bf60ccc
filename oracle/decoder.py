"""CPU restatement of the decoder prefill (TEST INFRASTRUCTURE ONLY: the
checker of the product's decoder, and bench.py's CPU baseline; never part of
the product path).

Composed from the pinned oracle functions of this package, in the order of
PhiDecoderLayer::forward (src/layer.cu:152-162):

    n1 = norm(x); q, k, v = Linear(n1)          (Linear::forward, src/layer.cu:18-25:
                                                 matmul_transposed, then + bias)
    q, k = apply_rope(q, k)                      (src/tensor.cu:191-210)
    a = attention(q, k, v)                       (src/layer.cu:115-141)
    h = o_proj(a) + x                            (src/layer.cu:155-156)
    y = MoE(norm(h)) + h                         (src/layer.cu:157-160)

and of the model: embedding rows, the layers, the final norm and lm_head on
the last row of every sequence (PhiTinyMoEModel::generate,
src/model.cu:1575-2059).  `cfg` is any object with DecoderConfig's fields;
`W` holds numpy arrays under the names random_weights gives them.
"""
from __future__ import annotations

import numpy as np

from . import (ACT_SWIGLU, attention, layer_norm, matmul_nt, moe_forward, rms_norm, rope)


def linear(x, w, b, contract):
    """Linear::forward: x W^T, then bias added row by row (add_bias_inplace)."""
    y = matmul_nt(x, w, contract)
    return y if b is None else (y + b[None, :]).astype(np.float32)


def norm(x, w, b, cfg):
    if cfg.norm == "rms":
        return rms_norm(x, w, cfg.norm_eps, cfg.contract)[0]
    return layer_norm(x, w, b, cfg.norm_eps, cfg.contract)[0]


def attention_block(x, L, cfg, batch, seq_len):
    """h = x + o_proj(attention(rope(q, k), v)) over norm(x)."""
    c = cfg
    n1 = norm(x, L["input_norm_w"], L["input_norm_b"], c)
    q = linear(n1, L["q_w"], L["q_b"], c.contract)
    k = linear(n1, L["k_w"], L["k_b"], c.contract)
    v = linear(n1, L["v_w"], L["v_b"], c.contract)
    q, k = rope(q, k, batch, seq_len, c.heads, c.kv_heads, c.head_dim, c.rope_theta)
    a = attention(q, k, v, batch, seq_len, c.heads, c.kv_heads, c.head_dim,
                  c.window if c.window > 0 else None)
    return (linear(a, L["o_w"], L["o_b"], c.contract) + x).astype(np.float32)


def moe_block(h, L, cfg):
    """y = h + MoE(norm(h)); returns (y, topk_idx, topk_w)."""
    c = cfg
    hn = norm(h, L["post_norm_w"], L["post_norm_b"], c)
    f, idx, w = moe_forward(hn, L["gate_w"], L["w1"], L["w3"], L["w2"], c.top_k,
                            act=ACT_SWIGLU, router_mode=c.router, contract=c.contract)
    return (f + h).astype(np.float32), idx, w


def layer_forward(x, L, cfg, batch, seq_len):
    """One decoder layer; returns (y, h, topk_idx) with h the MoE block's input."""
    h = attention_block(x, L, cfg, batch, seq_len)
    y, idx, _ = moe_block(h, L, cfg)
    return y, h, idx


def generate(tokens, W, cfg):
    """Logits [batch, vocab] of the last position of every sequence, and the
    per-layer (input, MoE-block input, routing) for diagnosis."""
    tokens = np.asarray(tokens)
    batch, seq_len = tokens.shape
    x = W["embed"][tokens.reshape(-1)].astype(np.float32)
    trace = []
    for L in W["layers"]:
        y, h, idx = layer_forward(x, L, cfg, batch, seq_len)
        trace.append((x, h, idx))
        x = y
    last = x[np.arange(1, batch + 1) * seq_len - 1]
    xn = norm(last, W["final_norm_w"], W["final_norm_b"], cfg)
    return linear(xn, W["lm_head_w"], W["lm_head_b"], cfg.contract), x, trace
