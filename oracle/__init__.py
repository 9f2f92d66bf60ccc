"""ctypes wrapper of the CPU oracle (oracle/moe_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as the
checker and by bench.py's cpu_baseline leg.  The product path never imports it.

Each function mirrors one piece of the reference CPU path; the C file cites
the reference file:line for each.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_moe.so")

CONTRACT_NONE = 0
CONTRACT_FMA = 1
ROUTER_PHI_QUANT = 0
ROUTER_SOFTMAX_TOPK = 1
ACT_SWIGLU = 0
ACT_SILU_MLP = 1

_lib = None


def build(force: bool = False) -> str:
    """Compile liboracle_moe.so with oracle/Makefile."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "-s", "-C", HERE],
                       check=True)
    return LIB_PATH


def build_native(out_dir: str) -> str:
    """Compile the oracle for this host's CPU (-march=native, the reference
    Makefile's host flags) into out_dir and return the library's path.
    Raises CalledProcessError when the host has no working gcc."""
    out = os.path.join(out_dir, "liboracle_moe_native.so")
    subprocess.run(["make", "-s", "-B", "-C", HERE, "MARCH=native", f"OUT={out}"],
                   check=True, capture_output=True)
    return out


def lib(path: str = None):
    """The loaded oracle library: the prebuilt one, or `path` when given on
    the first call (bench.py's native build).  A later call with another
    path is an error: ctypes keeps the first library loaded."""
    global _lib
    if _lib is not None and path is not None and path != _lib._name:
        raise RuntimeError(f"oracle already loaded from {_lib._name}")
    if _lib is None:
        if path is None:
            path = LIB_PATH
            if not os.path.exists(path):
                build()
        L = ctypes.CDLL(path)
        P = ctypes.c_void_p
        S = ctypes.c_size_t
        I = ctypes.c_int
        F = ctypes.c_float
        L.orc_lcg_fill.argtypes = [P, S, ctypes.c_uint32]
        L.orc_lcg_fill.restype = None
        for name in ("orc_matmul_nt", "orc_matmul_nn"):
            getattr(L, name).argtypes = [P, P, P, S, S, S, I]
            getattr(L, name).restype = I
        L.orc_silu.argtypes = [P, P, S]
        L.orc_silu.restype = None
        L.orc_mul.argtypes = [P, P, P, S]
        L.orc_mul.restype = None
        L.orc_layer_norm.argtypes = [P, P, P, F, S, S, I, P, P, P]
        L.orc_layer_norm.restype = I
        L.orc_rms_norm.argtypes = [P, P, F, S, S, I, P, P]
        L.orc_rms_norm.restype = I
        L.orc_rope_table.argtypes = [F, S, S, P]
        L.orc_rope_table.restype = I
        L.orc_rope.argtypes = [P, P, P, S, S, S, S, S]
        L.orc_rope.restype = I
        L.orc_attention.argtypes = [P, P, P, P, S, S, S, S, S, S]
        L.orc_attention.restype = I
        L.orc_route.argtypes = [P, P, S, S, S, I, F, F, P, P]
        L.orc_route.restype = I
        L.orc_permute.argtypes = [P, S, S, S, P, P, P]
        L.orc_permute.restype = I
        L.orc_expert_ffn.argtypes = [P, S, S, P, P, S, P, P, P, S, I, I, P]
        L.orc_expert_ffn.restype = I
        L.orc_combine.argtypes = [P, P, P, P, S, S, S, I, P]
        L.orc_combine.restype = I
        L.orc_moe_forward.argtypes = [P, S, S, P, P, S, S, P, P, P, S, I, I,
                                      F, F, I, P, P, P]
        L.orc_moe_forward.restype = I
        L.orc_set_threads.argtypes = [I]
        L.orc_set_threads.restype = None
        L.orc_get_threads.argtypes = []
        L.orc_get_threads.restype = I
        _lib = L
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _check(rc, what):
    if rc != 0:
        raise ValueError(f"oracle {what} failed (rc={rc})")


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def get_threads() -> int:
    return int(lib().orc_get_threads())


def lcg_fill(shape, seed: int) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    lib().orc_lcg_fill(_p(out), out.size, ctypes.c_uint32(seed))
    return out


def matmul_nt(a, b, contract=CONTRACT_FMA):
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    n = b.shape[0]
    assert b.shape[1] == k
    c = np.empty((m, n), dtype=np.float32)
    _check(lib().orc_matmul_nt(_p(a), _p(b), _p(c), m, n, k, contract), "matmul_nt")
    return c


def matmul_nn(a, b, contract=CONTRACT_FMA):
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    n = b.shape[1]
    assert b.shape[0] == k
    c = np.empty((m, n), dtype=np.float32)
    _check(lib().orc_matmul_nn(_p(a), _p(b), _p(c), m, n, k, contract), "matmul_nn")
    return c


def silu(x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().orc_silu(_p(x), _p(y), x.size)
    return y


def mul(a, b):
    a, b = _f32(a), _f32(b)
    c = np.empty_like(a)
    lib().orc_mul(_p(a), _p(b), _p(c), a.size)
    return c


def layer_norm(x, weight, bias, eps=1e-5, contract=CONTRACT_FMA):
    """tensor_ops::layer_norm over the last axis; returns (y, row_mean, row_inv)."""
    x, weight, bias = _f32(x), _f32(weight), _f32(bias)
    h = x.shape[-1]
    rows = x.size // h if h else 0
    assert weight.size == h and bias.size == h
    y = np.empty_like(x)
    mean = np.empty(rows, np.float32)
    inv = np.empty(rows, np.float32)
    _check(lib().orc_layer_norm(_p(x), _p(weight), _p(bias), float(eps), rows, h,
                                int(contract), _p(y), _p(mean), _p(inv)), "layer_norm")
    return y, mean, inv


def rope(q, k, batch, seq_len, q_heads, kv_heads, head_dim, theta=10000.0, table=None):
    """tensor_ops::apply_rope on copies of q [B*S, Hq*hd] and k [B*S, Hkv*hd]
    (table: rope_table(theta, head_dim, seq_len) unless given)."""
    q, k = _f32(q).copy(), _f32(k).copy()
    t = rope_table(theta, head_dim, seq_len) if table is None else _f32(table)
    _check(lib().orc_rope(_p(q), _p(k), _p(t), batch, seq_len, q_heads, kv_heads,
                          head_dim), "rope")
    return q, k


def rope_table(theta, head_dim, positions):
    """cos/sin of RoPE, [positions, head_dim/2, 2] (float libm calls)."""
    t = np.empty((positions, head_dim // 2, 2), np.float32)
    _check(lib().orc_rope_table(float(theta), head_dim, positions, _p(t)), "rope_table")
    return t


def attention(q, k, v, batch, seq_len, q_heads, kv_heads, head_dim, window=None):
    """PhiAttention's core (after the projections and RoPE): [B*S, Hq*hd]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.empty(q.shape, np.float32)
    w = seq_len if window is None else window
    _check(lib().orc_attention(_p(q), _p(k), _p(v), _p(out), batch, seq_len, q_heads,
                               kv_heads, head_dim, w), "attention")
    return out


def rms_norm(x, weight, eps=1e-5, contract=CONTRACT_FMA):
    """RMS norm over the last axis; returns (y, row_inv)."""
    x, weight = _f32(x), _f32(weight)
    h = x.shape[-1]
    rows = x.size // h if h else 0
    assert weight.size == h
    y = np.empty_like(x)
    inv = np.empty(rows, np.float32)
    _check(lib().orc_rms_norm(_p(x), _p(weight), float(eps), rows, h, int(contract), _p(y),
                              _p(inv)), "rms_norm")
    return y, inv


def route(logits, k, mode=ROUTER_PHI_QUANT, quantum=1e-3, tie_eps=2e-2,
          expert_bias=None):
    logits = _f32(logits)
    T, E = logits.shape
    bias = None if expert_bias is None else _f32(expert_bias)
    idx = np.empty((T, k), dtype=np.int32)
    w = np.empty((T, k), dtype=np.float32)
    _check(lib().orc_route(_p(logits), _p(bias), T, E, k, mode,
                           ctypes.c_float(quantum), ctypes.c_float(tie_eps),
                           _p(idx), _p(w)), "route")
    return idx, w


def permute(topk_idx, E):
    topk_idx = _i32(topk_idx)
    T, k = topk_idx.shape
    offsets = np.empty(E + 1, dtype=np.int32)
    perm = np.empty(max(T * k, 1), dtype=np.int32)
    inv = np.empty(max(T * k, 1), dtype=np.int32)
    _check(lib().orc_permute(_p(topk_idx), T, k, E, _p(offsets), _p(perm),
                             _p(inv)), "permute")
    return offsets, perm[:T * k], inv[:T * k].reshape(T, k)


def expert_ffn(x, perm, offsets, w1, w3, w2, act=ACT_SWIGLU,
               contract=CONTRACT_FMA):
    x, perm, offsets = _f32(x), _i32(perm), _i32(offsets)
    w1, w2 = _f32(w1), _f32(w2)
    w3 = None if w3 is None else _f32(w3)
    T, d = x.shape
    E, d_ff, _ = w1.shape
    out = np.zeros((max(int(offsets[-1]), 1), d), dtype=np.float32)
    _check(lib().orc_expert_ffn(_p(x), T, d, _p(perm), _p(offsets), E, _p(w1),
                                _p(w3), _p(w2), d_ff, act, contract, _p(out)),
           "expert_ffn")
    return out[:int(offsets[-1])]


def combine(out_rows, topk_idx, topk_w, inv, contract=CONTRACT_FMA):
    out_rows, topk_idx, topk_w, inv = (_f32(out_rows), _i32(topk_idx),
                                       _f32(topk_w), _i32(inv))
    T, k = topk_idx.shape
    d = out_rows.shape[1]
    y = np.empty((T, d), dtype=np.float32)
    _check(lib().orc_combine(_p(out_rows), _p(topk_idx), _p(topk_w), _p(inv),
                             T, k, d, contract, _p(y)), "combine")
    return y


def moe_forward(x, gate_w, w1, w3, w2, k, act=ACT_SWIGLU,
                router_mode=ROUTER_PHI_QUANT, quantum=1e-3, tie_eps=2e-2,
                contract=CONTRACT_FMA, expert_bias=None):
    """Returns (y, topk_idx, topk_w)."""
    x, gate_w, w1, w2 = _f32(x), _f32(gate_w), _f32(w1), _f32(w2)
    w3 = None if w3 is None else _f32(w3)
    bias = None if expert_bias is None else _f32(expert_bias)
    T, d = x.shape
    E = gate_w.shape[0]
    d_ff = w1.shape[1]
    y = np.empty((T, d), dtype=np.float32)
    idx = np.empty((T, k), dtype=np.int32)
    w = np.empty((T, k), dtype=np.float32)
    _check(lib().orc_moe_forward(_p(x), T, d, _p(gate_w), _p(bias), E, k,
                                 _p(w1), _p(w3), _p(w2), d_ff, act,
                                 router_mode, ctypes.c_float(quantum),
                                 ctypes.c_float(tie_eps), contract, _p(y),
                                 _p(idx), _p(w)), "moe_forward")
    return y, idx, w
