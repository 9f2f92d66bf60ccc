"""Decoder prefill on the library's kernels: config 5's 4-layer MoE decoder.

The layer is PhiDecoderLayer::forward (src/layer.cu:152-162) with the
projections of PhiAttention::forward (src/layer.cu:111-143):

    h = x + o_proj(attention(rope(q_proj(n1(x)), k_proj(n1(x))), v_proj(n1(x))))
    y = h + MoE(n2(h))

and the model is PhiTinyMoEModel::generate (src/model.cu:1575-2059) without
its prefix trie: embedding gather, the layers over all batch * seq_len rows,
then the final norm and lm_head on the last row of every sequence only
(the rows whose logits the model returns).  Every step is one call of the C
ABI on the current torch stream; nothing here computes on the host.

Norms are RMS norms by default, as config 5 names (n1, n2 and the final
norm; "layer" selects the reference's layer norm with bias).  The MoE block
is one moe_layer_forward with the post-attention norm and the residual
folded in (norm = n2, residual = 1).
"""
from __future__ import annotations

from dataclasses import dataclass

from . import (ACT_SWIGLU, CONTRACT_FMA, NORM_LAYER, NORM_RMS, ROUTER_SOFTMAX_TOPK,
               make_desc)


@dataclass
class DecoderConfig:
    """Shape of the decoder; the defaults are config 5."""
    layers: int = 4
    d: int = 1024
    heads: int = 16
    kv_heads: int = 16
    head_dim: int = 64
    experts: int = 8
    top_k: int = 2
    d_ff: int = 2816
    vocab: int = 32000
    norm: str = "rms"            # "rms" or "layer" (with bias)
    norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    window: int = 0              # sliding window of attention, 0 = unlimited
    router: int = ROUTER_SOFTMAX_TOPK
    contract: int = CONTRACT_FMA

    def __post_init__(self):
        if self.norm not in ("rms", "layer"):
            raise ValueError(f"norm must be 'rms' or 'layer', not {self.norm!r}")
        if self.heads * self.head_dim != self.d:
            raise ValueError("heads * head_dim must equal d")
        if self.kv_heads < 1 or self.heads % self.kv_heads:
            raise ValueError("heads must be a multiple of kv_heads")


def random_weights(cfg: DecoderConfig, device, seed: int = 0, std: float = 0.02):
    """Seeded random-init weights of the decoder's shapes (there is no
    checkpoint): embedding N(0, 1), projections, router, experts and lm_head
    N(0, std), biases N(0, std), norm weights 1 + N(0, 0.1), norm biases
    N(0, 0.1).  Names follow the reference's model.bin tensors."""
    import torch
    g = torch.Generator(device=device).manual_seed(seed)

    def rn(*shape, scale=std):
        return torch.randn(shape, device=device, generator=g) * scale

    layer_norm = cfg.norm == "layer"
    qw, kw = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim

    def norm_params():
        return 1 + rn(cfg.d, scale=0.1), (rn(cfg.d, scale=0.1) if layer_norm else None)

    W = {"embed": rn(cfg.vocab, cfg.d, scale=1.0), "layers": []}
    for _ in range(cfg.layers):
        n1w, n1b = norm_params()
        n2w, n2b = norm_params()
        W["layers"].append({
            "input_norm_w": n1w, "input_norm_b": n1b,
            "q_w": rn(qw, cfg.d), "q_b": rn(qw),
            "k_w": rn(kw, cfg.d), "k_b": rn(kw),
            "v_w": rn(kw, cfg.d), "v_b": rn(kw),
            "o_w": rn(cfg.d, qw), "o_b": rn(cfg.d),
            "post_norm_w": n2w, "post_norm_b": n2b,
            "gate_w": rn(cfg.experts, cfg.d),
            "w1": rn(cfg.experts, cfg.d_ff, cfg.d),
            "w3": rn(cfg.experts, cfg.d_ff, cfg.d),
            "w2": rn(cfg.experts, cfg.d, cfg.d_ff),
        })
    W["final_norm_w"], W["final_norm_b"] = norm_params()
    W["lm_head_w"] = rn(cfg.vocab, cfg.d)
    W["lm_head_b"] = rn(cfg.vocab)
    return W


class DecoderModel:
    """The decoder on one Context.  Activation buffers are grow-only and
    owned here, so repeated calls allocate nothing once warmed up.

    prune_last: generate() runs the last layer's q projection, attention,
    o projection and MoE block on the last row of every sequence only --
    the rows the logits read -- while its norm, k and v still cover every
    row (the reference's last-layer pruning, src/model.cu:1889-1960)."""

    def __init__(self, ctx, cfg: DecoderConfig, weights: dict, prune_last: bool = True):
        self.ctx, self.cfg, self.W = ctx, cfg, weights
        self.prune_last = prune_last
        self._bufs = {}
        self._shape = None

    # ---- buffers
    def _buf(self, name, shape, dtype=None):
        import torch
        dtype = dtype or torch.float32
        n = 1
        for s in shape:
            n *= s
        t = self._bufs.get(name)
        if t is None or t.numel() < n or t.dtype != dtype:
            t = torch.empty(max(n, 1), dtype=dtype, device=f"cuda:{self.ctx.device}")
            self._bufs[name] = t
        return t[:n].view(*shape)

    def moe_desc(self, rows):
        c = self.cfg
        return make_desc(rows, c.d, c.experts, c.top_k, c.d_ff, act=ACT_SWIGLU, router=c.router,
                         contract=c.contract,
                         norm=NORM_RMS if c.norm == "rms" else NORM_LAYER,
                         norm_eps=c.norm_eps, residual=True)

    def reserve(self, batch, seq_len):
        """Sizes every buffer and the context's workspace for batch x seq_len."""
        c, T = self.cfg, batch * seq_len
        for name in ("xa", "xb", "xn", "h"):
            self._buf(name, (T, c.d))
        self._buf("q", (T, c.heads * c.head_dim))
        self._buf("attn", (T, c.heads * c.head_dim))
        self._buf("k", (T, c.kv_heads * c.head_dim))
        self._buf("v", (T, c.kv_heads * c.head_dim))
        self.ctx.reserve(self.moe_desc(T))
        self.ctx.rope_table(c.rope_theta, c.head_dim, seq_len)
        self._last_rows(batch, seq_len)

    def _norm(self, x, w, b, y):
        c = self.cfg
        if c.norm == "rms":
            self.ctx.rms_norm(x, w, y=y, eps=c.norm_eps, contract=c.contract)
        else:
            self.ctx.layer_norm(x, w, b, y=y, eps=c.norm_eps, contract=c.contract)
        return y

    # ---- one layer
    def layer_forward(self, li, x, y, batch, seq_len, topk_idx=None, topk_w=None):
        """y = decoder layer li applied to x [batch*seq_len, d]."""
        c, ctx, L = self.cfg, self.ctx, self.W["layers"][li]
        T = batch * seq_len
        xn, h = self._buf("xn", (T, c.d)), self._buf("h", (T, c.d))
        q = self._buf("q", (T, c.heads * c.head_dim))
        k = self._buf("k", (T, c.kv_heads * c.head_dim))
        v = self._buf("v", (T, c.kv_heads * c.head_dim))
        attn = self._buf("attn", (T, c.heads * c.head_dim))
        self._norm(x, L["input_norm_w"], L["input_norm_b"], xn)
        ctx.sgemm_nt(xn, L["q_w"], q, bias=L["q_b"])
        ctx.sgemm_nt(xn, L["k_w"], k, bias=L["k_b"])
        ctx.sgemm_nt(xn, L["v_w"], v, bias=L["v_b"])
        ctx.rope(q, k, batch, seq_len, c.heads, c.kv_heads, c.head_dim, c.rope_theta,
                 table=ctx.rope_table(c.rope_theta, c.head_dim, seq_len))
        ctx.attention(q, k, v, attn, batch, seq_len, c.heads, c.kv_heads, c.head_dim,
                      c.window)
        # h = o_proj(attn) + x (the reference's add_inplace(attn, x)), the
        # residual added in the GEMM's store
        ctx.sgemm_nt(attn, L["o_w"], h, bias=L["o_b"], residual=x)
        moe = {"gate_w": L["gate_w"], "w1": L["w1"], "w3": L["w3"], "w2": L["w2"],
               "norm_w": L["post_norm_w"], "norm_b": L["post_norm_b"]}
        ctx.layer_forward(self.moe_desc(T), moe, h, y, topk_idx, topk_w)
        return y

    def _last_rows(self, batch, seq_len):
        """Row indices b * seq_len + seq_len - 1 of the last position of every
        sequence, on the device (rebuilt when the shape changes)."""
        import torch
        last = self._buf("last_idx", (batch,), torch.int32)
        if self._shape != (batch, seq_len):
            last.copy_(torch.arange(1, batch + 1, dtype=torch.int32) * seq_len - 1)
            self._shape = (batch, seq_len)
        return last

    def last_layer_tail(self, li, x, y_last, batch, seq_len, topk_idx=None):
        """Layer li on the last rows only: y_last [batch, d] = the layer's
        output rows b * seq_len + seq_len - 1 of x [batch*seq_len, d]."""
        c, ctx, L = self.cfg, self.ctx, self.W["layers"][li]
        T = batch * seq_len
        qw, kw = c.heads * c.head_dim, c.kv_heads * c.head_dim
        xn = self._buf("xn", (T, c.d))
        k, v = self._buf("k", (T, kw)), self._buf("v", (T, kw))
        last = self._last_rows(batch, seq_len)
        xn_l, x_l = self._buf("tail_xn", (batch, c.d)), self._buf("tail_x", (batch, c.d))
        q_l, a_l = self._buf("tail_q", (batch, qw)), self._buf("tail_attn", (batch, qw))
        h_l = self._buf("tail_h", (batch, c.d))
        self._norm(x, L["input_norm_w"], L["input_norm_b"], xn)
        ctx.sgemm_nt(xn, L["k_w"], k, bias=L["k_b"])
        ctx.sgemm_nt(xn, L["v_w"], v, bias=L["v_b"])
        ctx.embed(xn, last, xn_l)  # row gathers of the last rows
        ctx.embed(x, last, x_l)
        ctx.sgemm_nt(xn_l, L["q_w"], q_l, bias=L["q_b"])
        table = ctx.rope_table(c.rope_theta, c.head_dim, seq_len)
        ctx.rope(None, k, batch, seq_len, 0, c.kv_heads, c.head_dim, table=table)
        ctx.rope(q_l, None, batch, 1, c.heads, 0, c.head_dim, table=table, first_pos=seq_len - 1)
        ctx.attention_last(q_l, k, v, a_l, batch, seq_len, c.heads, c.kv_heads, c.head_dim,
                           c.window)
        ctx.sgemm_nt(a_l, L["o_w"], h_l, bias=L["o_b"], residual=x_l)
        moe = {"gate_w": L["gate_w"], "w1": L["w1"], "w3": L["w3"], "w2": L["w2"],
               "norm_w": L["post_norm_w"], "norm_b": L["post_norm_b"]}
        ctx.layer_forward(self.moe_desc(batch), moe, h_l, y_last, topk_idx)
        return y_last

    # ---- the model
    def hidden(self, tokens, routing=None, layers=None):
        """The residual stream after the first `layers` layers (all by
        default), [batch*seq_len, d].  routing: a list that receives each
        layer's top-k experts [T, k]."""
        import torch
        batch, seq_len = tokens.shape
        T = batch * seq_len
        tok = tokens.reshape(-1)
        if tok.dtype != torch.int32 or not tok.is_contiguous():
            tok = tok.to(torch.int32).contiguous()
        x, y = self._buf("xa", (T, self.cfg.d)), self._buf("xb", (T, self.cfg.d))
        self.ctx.embed(self.W["embed"], tok, x)
        for li in range(self.cfg.layers if layers is None else layers):
            idx = None
            if routing is not None:
                idx = torch.empty((T, self.cfg.top_k), dtype=torch.int32, device=x.device)
                routing.append(idx)
            self.layer_forward(li, x, y, batch, seq_len, topk_idx=idx)
            x, y = y, x
        return x

    def generate(self, tokens, logits=None, routing=None):
        """Logits [batch, vocab] of the last position of every sequence of
        tokens [batch, seq_len] (int32, on the device).  routing receives
        each layer's top-k experts (the pruned last layer's: [batch, k])."""
        import torch
        batch, seq_len = tokens.shape
        c = self.cfg
        xl = self._buf("xl", (batch, c.d))
        xln = self._buf("xln", (batch, c.d))
        if self.prune_last and c.layers > 0:
            x = self.hidden(tokens, routing, layers=c.layers - 1)
            idx = None
            if routing is not None:
                idx = torch.empty((batch, c.top_k), dtype=torch.int32, device=x.device)
                routing.append(idx)
            self.last_layer_tail(c.layers - 1, x, xl, batch, seq_len, topk_idx=idx)
        else:
            x = self.hidden(tokens, routing)
            self.ctx.embed(x, self._last_rows(batch, seq_len), xl)  # the last rows
        self._norm(xl, self.W["final_norm_w"], self.W["final_norm_b"], xln)
        if logits is None:
            logits = torch.empty((batch, c.vocab), device=x.device)
        self.ctx.sgemm_nt(xln, self.W["lm_head_w"], logits, bias=self.W["lm_head_b"])
        return logits


class CapturedPrefill:
    """One generate() of a fixed (batch, seq_len) captured in a HIP graph:
    replay() reruns every kernel of the prefill on `tokens` (update it in
    place) into `logits` with one launch from the host.

    The capture runs on a Context of its own, so no other call can grow
    (and free) the workspace the graph's kernels address, and the graph
    keeps its activation buffers alive.  The library records no memset and
    makes no host synchronisation inside a step once its workspace is sized
    (one eager warm-up call does that here)."""

    def __init__(self, model: DecoderModel, batch: int, seq_len: int, warmup: int = 1):
        import torch
        from . import Context
        self.ctx = Context(model.ctx.device)
        self.model = DecoderModel(self.ctx, model.cfg, model.W, prune_last=model.prune_last)
        self.model.reserve(batch, seq_len)
        dev = f"cuda:{model.ctx.device}"
        self.tokens = torch.zeros((batch, seq_len), dtype=torch.int32, device=dev)
        self.logits = torch.empty((batch, model.cfg.vocab), device=dev)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(max(warmup, 1)):
                self.model.generate(self.tokens, self.logits)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.model.generate(self.tokens, self.logits)
        torch.cuda.synchronize()

    def replay(self, tokens=None):
        if tokens is not None:
            self.tokens.copy_(tokens)
        self.graph.replay()
        return self.logits

    def close(self):
        self.graph = None
        self.ctx.close()
