"""Python binding of the gfx950 MoE library (libmoe_amd.so) over its C ABI.

The functions mirror the entry points declared in include/moe_amd.h and the
reference operators they replace (tensor_ops::matmul_transposed,
PhiMoE::route, PhiMoE::forward ...).  Arguments are torch tensors on the GPU;
work is enqueued on torch's current stream.  There is no fallback: if the
HIP library is missing or fails to load, every call raises.

Load it by path, as a package (the directory name is not a Python
identifier; decoder.py beside this file is its submodule):

    spec = importlib.util.spec_from_file_location(
        "moe_amd", "accelerating-moe-inference_amd/__init__.py",
        submodule_search_locations=["accelerating-moe-inference_amd"])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["moe_amd"] = mod
    spec.loader.exec_module(mod)
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmoe_amd.so")

OK, ERR_INVALID, ERR_RUNTIME, ERR_UNSUPPORTED = 0, 1, 2, 3
CONTRACT_NONE, CONTRACT_FMA = 0, 1
ROUTER_PHI_QUANT, ROUTER_SOFTMAX_TOPK = 0, 1
ACT_SWIGLU, ACT_SILU_MLP = 0, 1
NORM_NONE, NORM_LAYER, NORM_RMS = 0, 1, 2

EXPORTS = (
    "moe_ctx_create", "moe_ctx_destroy", "moe_ctx_reserve", "moe_ctx_set_timing",
    "moe_ctx_kernel_times", "moe_ctx_reset_timing", "moe_last_error",
    "moe_version", "moe_sgemm_nt", "moe_sgemm_nn", "moe_sgemm_nt_residual", "moe_silu",
    "moe_mul",
    "moe_layer_norm", "moe_rms_norm", "moe_rope_table", "moe_rope", "moe_attention",
    "moe_attention_last", "moe_rope_rows", "moe_attention_paths", "moe_add",
    "moe_add_bias", "moe_embed", "moe_gate_logits",
    "moe_route", "moe_permute", "moe_expert_ffn_grouped", "moe_combine",
    "moe_layer_forward", "moe_layer_forward_noalloc", "moe_layer_w2_splits",
    "moe_ctx_set_stream_k", "moe_ctx_workspace_bytes", "moe_launch_floor", "moe_sgemm_plan",
)


class MoeInvalidArgument(ValueError):
    """MOE_ERR_INVALID (std::invalid_argument in the C++ drop-in)."""


class MoeRuntimeError(RuntimeError):
    """MOE_ERR_RUNTIME / MOE_ERR_UNSUPPORTED (std::runtime_error)."""


class LayerDesc(ctypes.Structure):
    _fields_ = [("T", ctypes.c_int64), ("d", ctypes.c_int64),
                ("E", ctypes.c_int64), ("k", ctypes.c_int64),
                ("d_ff", ctypes.c_int64), ("act", ctypes.c_int32),
                ("router", ctypes.c_int32), ("quantum", ctypes.c_float),
                ("tie_eps", ctypes.c_float), ("contract", ctypes.c_int32),
                ("norm", ctypes.c_int32), ("norm_eps", ctypes.c_float),
                ("residual", ctypes.c_int32)]


class LayerWeights(ctypes.Structure):
    _fields_ = [("gate_w", ctypes.c_void_p), ("expert_bias", ctypes.c_void_p),
                ("w1", ctypes.c_void_p), ("w3", ctypes.c_void_p),
                ("w2", ctypes.c_void_p), ("norm_w", ctypes.c_void_p),
                ("norm_b", ctypes.c_void_p)]


_lib = None


def load_library(path: str = LIB_PATH):
    """Loads libmoe_amd.so; raises if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: build it with "
            "`python accelerating-moe-inference_amd/build.py`")
    L = ctypes.CDLL(path)
    P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    F = ctypes.c_float
    sig = {
        "moe_ctx_create": ([I, ctypes.POINTER(P)], I),
        "moe_ctx_destroy": ([P], I),
        "moe_ctx_reserve": ([P, ctypes.POINTER(LayerDesc)], I),
        "moe_ctx_set_timing": ([P, I], I),
        "moe_ctx_kernel_times": ([P, ctypes.POINTER(ctypes.c_char_p),
                                  ctypes.POINTER(ctypes.c_double),
                                  ctypes.POINTER(ctypes.c_int64), I], I),
        "moe_ctx_reset_timing": ([P], I),
        "moe_last_error": ([], ctypes.c_char_p),
        "moe_version": ([], ctypes.c_char_p),
        "moe_sgemm_nt": ([P, P, P, P, P, I64, I64, I64, P], I),
        "moe_sgemm_nn": ([P, P, P, P, P, I64, I64, I64, P], I),
        "moe_sgemm_nt_residual": ([P, P, P, P, P, P, I64, I64, I64, P], I),
        "moe_silu": ([P, P, P, I64, P], I),
        "moe_mul": ([P, P, P, P, I64, P], I),
        "moe_layer_norm": ([P, P, P, P, F, I64, I64, I, P, P, P, P], I),
        "moe_rms_norm": ([P, P, P, F, I64, I64, I, P, P, P], I),
        "moe_rope_table": ([F, I64, I64, P], I),
        "moe_rope": ([P, P, P, P, I64, I64, I64, I64, I64, I64, I64, P], I),
        "moe_attention_last": ([P, P, P, P, P, I64, I64, I64, I64, I64, I64, P], I),
        "moe_rope_rows": ([P, P, P, P, I64, P, I64, I64, I64, I64, P], I),
        "moe_attention_paths": ([P, P, P, P, P, I64, I64, P, P, P, I64, I64, I64, I64, I64,
                                 I64, P], I),
        "moe_attention": ([P, P, P, P, P, I64, I64, I64, I64, I64, I64, P], I),
        "moe_add": ([P, P, P, I64, P], I),
        "moe_add_bias": ([P, P, P, I64, I64, P], I),
        "moe_embed": ([P, P, P, I64, I64, I64, P, P], I),
        "moe_gate_logits": ([P, P, P, P, I64, I64, I64, I, P], I),
        "moe_route": ([P, P, P, I64, I64, I64, I, F, F, P, P, P], I),
        "moe_permute": ([P, P, I64, I64, I64, P, P, P, P], I),
        "moe_expert_ffn_grouped": ([P, P, P, P, P, P, P, I, I64, I64, I64,
                                    I64, I64, P, P, P], I),
        "moe_combine": ([P, P, P, P, P, P, P, I64, I64, I64, I, P], I),
        "moe_layer_forward": ([P, ctypes.POINTER(LayerDesc),
                               ctypes.POINTER(LayerWeights), P, P, P, P, P], I),
        "moe_layer_forward_noalloc": ([P, ctypes.POINTER(LayerDesc),
                                       ctypes.POINTER(LayerWeights), P, P, P, P, P], I),
        "moe_layer_w2_splits": ([P, ctypes.POINTER(LayerDesc), ctypes.POINTER(ctypes.c_int32)],
                                I),
        "moe_ctx_set_stream_k": ([P, I], I),
        "moe_ctx_workspace_bytes": ([P, ctypes.POINTER(ctypes.c_int64)], I),
        "moe_launch_floor": ([P, P], I),
        "moe_sgemm_plan": ([P, I, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                            ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32)], I),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


def _check(rc: int) -> None:
    if rc == OK:
        return
    msg = _lib.moe_last_error().decode()
    if rc == ERR_INVALID:
        raise MoeInvalidArgument(msg)
    raise MoeRuntimeError(f"[{rc}] {msg}")


def _ptr(t):
    if t is None:
        return None
    if not t.is_cuda:
        raise MoeInvalidArgument("tensor must be on the GPU")
    if not t.is_contiguous():
        raise MoeInvalidArgument("tensor must be contiguous")
    return ctypes.c_void_p(t.data_ptr())


def _f32(t, name):
    import torch
    if t is not None and t.dtype != torch.float32:
        raise MoeInvalidArgument(f"{name} must be float32")
    return _ptr(t)


def _i32(t, name):
    import torch
    if t is not None and t.dtype != torch.int32:
        raise MoeInvalidArgument(f"{name} must be int32")
    return _ptr(t)


def _stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


class Context:
    """A moe_ctx bound to one device (workspace + optional kernel timing)."""

    def __init__(self, device: int = 0):
        L = load_library()
        h = ctypes.c_void_p()
        _check(L.moe_ctx_create(device, ctypes.byref(h)))
        self.handle = h
        self.device = device
        self._rope_tables = {}

    def close(self):
        if self.handle:
            _check(_lib.moe_ctx_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- timing
    def set_timing(self, on: bool):
        _check(_lib.moe_ctx_set_timing(self.handle, 1 if on else 0))

    def reset_timing(self):
        _check(_lib.moe_ctx_reset_timing(self.handle))

    def kernel_times(self):
        """{kernel name: (total ms, launches)} since the last reset."""
        cap = 64
        names = (ctypes.c_char_p * cap)()
        ms = (ctypes.c_double * cap)()
        n = (ctypes.c_int64 * cap)()
        cnt = _lib.moe_ctx_kernel_times(self.handle, names, ms, n, cap)
        if cnt < 0:
            _check(-cnt)
        return {names[i].decode(): (ms[i], n[i]) for i in range(min(cnt, cap))}

    def reserve(self, desc: LayerDesc):
        _check(_lib.moe_ctx_reserve(self.handle, ctypes.byref(desc)))

    def workspace_bytes(self) -> int:
        """moe_ctx_workspace_bytes: the context's workspace as it stands."""
        out = ctypes.c_int64(0)
        _check(_lib.moe_ctx_workspace_bytes(self.handle, ctypes.byref(out)))
        return out.value

    def launch_floor(self):
        """moe_launch_floor: one empty kernel on the current stream (timed
        as "empty" when timing is on)."""
        _check(_lib.moe_launch_floor(self.handle, _stream()))

    # ---- operators
    def sgemm_nt(self, A, B, C, bias=None, residual=None):
        """C = A B^T (+ bias) (+ residual, added after the bias in the same
        kernel; residual may be C itself)."""
        M, K = A.shape
        N = B.shape[0]
        if residual is None:
            _check(_lib.moe_sgemm_nt(self.handle, _f32(A, "A"), _f32(B, "B"),
                                     _f32(bias, "bias"), _f32(C, "C"), M, N, K,
                                     _stream()))
        else:
            if tuple(residual.shape) != (M, N):
                raise ValueError(f"residual shape {tuple(residual.shape)} != {(M, N)}")
            _check(_lib.moe_sgemm_nt_residual(self.handle, _f32(A, "A"), _f32(B, "B"),
                                              _f32(bias, "bias"), _f32(residual, "residual"),
                                              _f32(C, "C"), M, N, K, _stream()))
        return C

    def sgemm_nn(self, A, B, C, bias=None):
        M, K = A.shape
        N = B.shape[1]
        _check(_lib.moe_sgemm_nn(self.handle, _f32(A, "A"), _f32(B, "B"),
                                 _f32(bias, "bias"), _f32(C, "C"), M, N, K,
                                 _stream()))
        return C

    def silu(self, x, y):
        _check(_lib.moe_silu(self.handle, _f32(x, "x"), _f32(y, "y"), x.numel(),
                             _stream()))
        return y

    def mul(self, a, b, c):
        _check(_lib.moe_mul(self.handle, _f32(a, "a"), _f32(b, "b"), _f32(c, "c"),
                            a.numel(), _stream()))
        return c

    def layer_norm(self, x, weight, bias, y=None, eps=1e-5, contract=CONTRACT_FMA,
                   row_mean=None, row_inv=None):
        """Layer norm over the last axis; y / row_mean / row_inv may be None."""
        h = x.shape[-1]
        rows = x.numel() // h if h else 0
        _check(_lib.moe_layer_norm(self.handle, _f32(x, "x"), _f32(weight, "weight"),
                                   _f32(bias, "bias"), eps, rows, h, contract,
                                   _f32(y, "y"), _f32(row_mean, "row_mean"),
                                   _f32(row_inv, "row_inv"), _stream()))
        return y

    def rms_norm(self, x, weight, y=None, eps=1e-5, contract=CONTRACT_FMA, row_inv=None):
        """RMS norm over the last axis; y / row_inv may be None."""
        h = x.shape[-1]
        rows = x.numel() // h if h else 0
        _check(_lib.moe_rms_norm(self.handle, _f32(x, "x"), _f32(weight, "weight"), eps, rows,
                                 h, contract, _f32(y, "y"), _f32(row_inv, "row_inv"), _stream()))
        return y

    def rope_table(self, theta, head_dim, positions):
        """The cos/sin table [positions, head_dim/2, 2] on this context's
        device, built on the host by moe_rope_table (cached per shape)."""
        import numpy as np
        import torch
        key = (float(theta), int(head_dim), int(positions))
        t = self._rope_tables.get(key)
        if t is None:
            host = np.empty(max(positions * head_dim, 1), np.float32)
            _check(_lib.moe_rope_table(float(theta), head_dim, positions,
                                       host.ctypes.data_as(ctypes.c_void_p)))
            t = torch.from_numpy(host).to(f"cuda:{self.device}")
            self._rope_tables[key] = t
        return t

    def rope(self, q, k, batch, seq_len, q_heads, kv_heads, head_dim, theta=10000.0,
             table=None, first_pos=0):
        """RoPE in place on q [B*S, Hq*hd] and k [B*S, Hkv*hd]; row r at
        position first_pos + r % seq_len."""
        if table is None:
            table = self.rope_table(theta, head_dim, first_pos + seq_len)
        positions = table.numel() // head_dim if head_dim else 0
        _check(_lib.moe_rope(self.handle, _f32(q, "q"), _f32(k, "k"), _f32(table, "table"),
                             positions, batch, seq_len, first_pos, q_heads, kv_heads, head_dim,
                             _stream()))

    def attention(self, q, k, v, out, batch, seq_len, q_heads, kv_heads, head_dim, window=0):
        """Causal attention per sequence and head; window 0 = unlimited."""
        _check(_lib.moe_attention(self.handle, _f32(q, "q"), _f32(k, "k"), _f32(v, "v"),
                                  _f32(out, "out"), batch, seq_len, q_heads, kv_heads,
                                  head_dim, window, _stream()))
        return out

    def attention_last(self, q, k, v, out, batch, seq_len, q_heads, kv_heads, head_dim,
                       window=0):
        """Attention of the last position of each sequence: q and out
        [batch, Hq*hd], k and v [batch*seq_len, Hkv*hd]."""
        _check(_lib.moe_attention_last(self.handle, _f32(q, "q"), _f32(k, "k"), _f32(v, "v"),
                                       _f32(out, "out"), batch, seq_len, q_heads, kv_heads,
                                       head_dim, window, _stream()))
        return out

    def rope_rows(self, q, k, table, positions, rows, q_heads, kv_heads, head_dim):
        """RoPE with row r at positions[r] (int32, on the device)."""
        _check(_lib.moe_rope_rows(self.handle, _f32(q, "q"), _f32(k, "k"), _f32(table, "table"),
                                  table.numel() // head_dim, _i32(positions, "positions"), rows,
                                  q_heads, kv_heads, head_dim, _stream()))

    def attention_paths(self, q, k, v, out, key_rows, key_beg, key_end, max_len, q_heads,
                        kv_heads, head_dim, window=0):
        """Attention of q's rows over explicit key lists (int32 device arrays)."""
        nq = key_beg.numel()
        _check(_lib.moe_attention_paths(
            self.handle, _f32(q, "q"), _f32(k, "k"), _f32(v, "v"), _f32(out, "out"), nq,
            k.shape[0], _i32(key_rows, "key_rows"), _i32(key_beg, "key_beg"),
            _i32(key_end, "key_end"), max_len, key_rows.numel(), q_heads, kv_heads, head_dim,
            window, _stream()))
        return out

    def add(self, a, b):
        """a += b."""
        _check(_lib.moe_add(self.handle, _f32(a, "a"), _f32(b, "b"), a.numel(), _stream()))
        return a

    def add_bias(self, a, bias):
        """a[r, c] += bias[c]."""
        cols = bias.numel()
        _check(_lib.moe_add_bias(self.handle, _f32(a, "a"), _f32(bias, "bias"),
                                 a.numel() // cols if cols else 0, cols, _stream()))
        return a

    def embed(self, table, tokens, out):
        """out[i] = table[tokens[i]]."""
        vocab, d = table.shape
        _check(_lib.moe_embed(self.handle, _f32(table, "table"), _i32(tokens, "tokens"),
                              tokens.numel(), d, vocab, _f32(out, "out"), _stream()))
        return out

    def gate_logits(self, x, gate_w, logits, contract=CONTRACT_FMA):
        T, d = x.shape
        E = gate_w.shape[0]
        _check(_lib.moe_gate_logits(self.handle, _f32(x, "x"),
                                    _f32(gate_w, "gate_w"),
                                    _f32(logits, "logits"), T, d, E, contract,
                                    _stream()))
        return logits

    def route(self, logits, k, topk_idx, topk_w, mode=ROUTER_PHI_QUANT,
              quantum=1e-3, tie_eps=2e-2, expert_bias=None):
        T, E = logits.shape
        _check(_lib.moe_route(self.handle, _f32(logits, "logits"),
                              _f32(expert_bias, "expert_bias"), T, E, k, mode,
                              quantum, tie_eps, _i32(topk_idx, "topk_idx"),
                              _f32(topk_w, "topk_w"), _stream()))
        return topk_idx, topk_w

    def permute(self, topk_idx, E, offsets, perm, inv):
        T, k = topk_idx.shape
        _check(_lib.moe_permute(self.handle, _i32(topk_idx, "topk_idx"), T, k,
                                E, _i32(offsets, "offsets"), _i32(perm, "perm"),
                                _i32(inv, "inv"), _stream()))
        return offsets, perm, inv

    def expert_ffn_grouped(self, x, perm, offsets, w1, w3, w2, k, h, out_rows,
                           act=ACT_SWIGLU):
        T, d = x.shape
        E, d_ff, _ = w1.shape
        _check(_lib.moe_expert_ffn_grouped(
            self.handle, _f32(x, "x"), _i32(perm, "perm"),
            _i32(offsets, "offsets"), _f32(w1, "w1"), _f32(w3, "w3"),
            _f32(w2, "w2"), act, T, k, d, d_ff, E, _f32(h, "h"),
            _f32(out_rows, "out_rows"), _stream()))
        return out_rows

    def combine(self, out_rows, topk_idx, topk_w, inv, y, resid=None,
                contract=CONTRACT_FMA):
        T, k = topk_idx.shape
        d = y.shape[1]
        _check(_lib.moe_combine(self.handle, _f32(out_rows, "out_rows"),
                                _i32(topk_idx, "topk_idx"),
                                _f32(topk_w, "topk_w"), _i32(inv, "inv"),
                                _f32(resid, "resid"), _f32(y, "y"), T, k, d,
                                contract, _stream()))
        return y

    def layer_forward(self, desc: LayerDesc, weights: dict, x, y,
                      topk_idx=None, topk_w=None, noalloc=False):
        """moe_layer_forward, or (noalloc) moe_layer_forward_noalloc: the same
        layer on the library's fixed per-GPU scratch, allocating nothing."""
        W = LayerWeights(
            gate_w=_f32(weights["gate_w"], "gate_w"),
            expert_bias=_f32(weights.get("expert_bias"), "expert_bias"),
            w1=_f32(weights["w1"], "w1"), w3=_f32(weights.get("w3"), "w3"),
            w2=_f32(weights["w2"], "w2"),
            norm_w=_f32(weights.get("norm_w"), "norm_w"),
            norm_b=_f32(weights.get("norm_b"), "norm_b"))
        fn = _lib.moe_layer_forward_noalloc if noalloc else _lib.moe_layer_forward
        _check(fn(self.handle, ctypes.byref(desc), ctypes.byref(W), _f32(x, "x"),
                  _f32(y, "y"), _i32(topk_idx, "topk_idx"), _f32(topk_w, "topk_w"),
                  _stream()))
        return y

    def set_stream_k(self, mode: int) -> None:
        """moe_ctx_set_stream_k: -1 planner, 0 one tile per workgroup, 1
        stream-K for the grouped expert GEMMs of this context."""
        _check(_lib.moe_ctx_set_stream_k(self.handle, int(mode)))

    def sgemm_plan(self, M: int, N: int, K: int, nn: bool = True) -> dict:
        """moe_sgemm_plan: the tile shape id and K splits moe_sgemm_nn /
        moe_sgemm_nt runs M x N x K with on this context's GPU."""
        t, sp = ctypes.c_int32(0), ctypes.c_int32(0)
        _check(_lib.moe_sgemm_plan(self.handle, int(bool(nn)), int(M), int(N), int(K),
                                   ctypes.byref(t), ctypes.byref(sp)))
        return {"tile": t.value, "splits": sp.value}

    def w2_splits(self, desc: LayerDesc) -> int:
        """K splits layer_forward(desc) uses for w2 on this context's GPU."""
        out = ctypes.c_int32(0)
        _check(_lib.moe_layer_w2_splits(self.handle, ctypes.byref(desc), ctypes.byref(out)))
        return out.value


def make_desc(T, d, E, k, d_ff, act=ACT_SWIGLU, router=ROUTER_PHI_QUANT,
              quantum=1e-3, tie_eps=2e-2, contract=CONTRACT_FMA, norm=NORM_NONE,
              norm_eps=1e-5, residual=False) -> LayerDesc:
    return LayerDesc(T=T, d=d, E=E, k=k, d_ff=d_ff, act=act, router=router,
                     quantum=quantum, tie_eps=tie_eps, contract=contract, norm=norm,
                     norm_eps=norm_eps, residual=int(bool(residual)))


from .decoder import DecoderConfig, DecoderModel, random_weights  # noqa: E402
