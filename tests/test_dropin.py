"""The C++ drop-in of the reference host API (Tensor, tensor_ops, ModelLoader,
Linear, PhiMLP, PhiMoE), driven through tests/cpp/dropin_shim.cpp.

CPU tests: Tensor semantics and every ModelLoader error path.  GPU tests:
each layer against the oracle on a model.bin written in the reference format
(src/model_loader.cu:14-30)."""
import ctypes
import os
import struct
import subprocess

import numpy as np
import pytest

from helpers import ROOT, assert_close, normal

SHIM_DIR = os.path.join(ROOT, "tests", "cpp")
SHIM = os.path.join(SHIM_DIR, "libdropin_shim.so")
INVALID, RUNTIME, LOGIC, OUT_OF_RANGE = 1, 2, 3, 4


@pytest.fixture(scope="module")
def shim():
    if not os.path.exists(SHIM):
        subprocess.run(["make", "-s", "-C", SHIM_DIR], check=True)
    L = ctypes.CDLL(SHIM)
    L.shim_error.restype = ctypes.c_char_p
    return L


def err(shim):
    return shim.shim_error().decode()


def write_model_bin(path, tensors):
    """model.bin: u32 count; per tensor u32 name_len, name, u32 ndim,
    u32 dims[ndim], u64 offset, u64 bytes; fp32 data at the offsets."""
    header = 4 + sum(4 + len(n.encode()) + 4 + 4 * a.ndim + 16 for n, a in tensors.items())
    blob = bytearray(struct.pack("<I", len(tensors)))
    off = header
    datas = []
    for name, a in tensors.items():
        a = np.ascontiguousarray(a, dtype=np.float32)
        nb = name.encode()
        blob += struct.pack("<I", len(nb)) + nb + struct.pack("<I", a.ndim)
        blob += struct.pack(f"<{a.ndim}I", *a.shape)
        blob += struct.pack("<QQ", off, a.nbytes)
        datas.append(a.tobytes())
        off += a.nbytes
    assert len(blob) == header
    with open(path, "wb") as f:
        f.write(bytes(blob))
        for d in datas:
            f.write(d)


def fptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------- CPU side
def test_tensor_semantics(shim):
    assert shim.shim_tensor_semantics(0) == 0, err(shim)


def test_loader_reads_shapes_and_values(shim, tmp_path):
    rng = np.random.default_rng(0)
    a = normal(rng, (3, 5))
    b = normal(rng, (7,))
    path = str(tmp_path / "model.bin")
    write_model_bin(path, {"a.weight": a, "layer.b": b})
    dims = (ctypes.c_int64 * 8)()
    nd = ctypes.c_int()
    assert shim.shim_loader_shape(path.encode(), b"a.weight", dims, ctypes.byref(nd)) == 0
    assert list(dims[:nd.value]) == [3, 5]
    out = np.empty(7, np.float32)
    assert shim.shim_loader_load(path.encode(), b"layer.b", fptr(out), ctypes.c_int64(7)) == 0
    assert np.array_equal(out, b)


def test_loader_error_paths(shim, tmp_path):
    path = str(tmp_path / "model.bin")
    write_model_bin(path, {"w": np.ones((2, 2), np.float32)})
    out = np.empty(4, np.float32)
    rc = shim.shim_loader_load(path.encode(), b"nope", fptr(out), ctypes.c_int64(4))
    assert rc == RUNTIME and err(shim) == "missing tensor: nope"
    rc = shim.shim_loader_load(str(tmp_path / "absent.bin").encode(), b"w", fptr(out),
                               ctypes.c_int64(4))
    assert rc == RUNTIME and err(shim).startswith("cannot open model")
    raw = open(path, "rb").read()
    trunc = str(tmp_path / "trunc_header.bin")
    open(trunc, "wb").write(raw[:10])
    rc = shim.shim_loader_load(trunc.encode(), b"w", fptr(out), ctypes.c_int64(4))
    assert rc == RUNTIME and err(shim) == "truncated model.bin"
    trunc = str(tmp_path / "trunc_data.bin")
    open(trunc, "wb").write(raw[:-4])
    rc = shim.shim_loader_load(trunc.encode(), b"w", fptr(out), ctypes.c_int64(4))
    assert rc == RUNTIME and err(shim) == "truncated tensor: w"
    # bytes field that is not 4 * elements: not fp32
    bad = bytearray(raw)
    hdr = 4 + 4 + 1 + 4 + 8
    bad[hdr + 8:hdr + 16] = struct.pack("<Q", 8)
    badp = str(tmp_path / "bad.bin")
    open(badp, "wb").write(bytes(bad))
    rc = shim.shim_loader_load(badp.encode(), b"w", fptr(out), ctypes.c_int64(4))
    assert rc == RUNTIME and err(shim) == "tensor is not float32: w"


def test_shape_errors_before_any_device_work(shim):
    assert shim.shim_matmul_bad_shape() == INVALID
    assert err(shim) == "matmul_transposed shape"
    assert shim.shim_outside_op() == LOGIC
    assert "never defined" in err(shim)
    want = {1: (INVALID, "add shape"), 2: (INVALID, "bias shape"), 3: (INVALID, "bias shape"),
            4: (INVALID, "apply_rope shape"), 5: (INVALID, "apply_rope shape"),
            6: (OUT_OF_RANGE, "Tensor index")}
    for which, (code, msg) in want.items():
        assert shim.shim_elementwise_bad_shape(which) == code, which
        assert err(shim) == msg
    assert shim.shim_layer_norm_bad_shape() == INVALID
    assert err(shim) == "layer norm shape"


def test_moe_timing_rejects_nonpositive_iterations(shim):
    x = np.zeros((2, 4), np.float32)
    I = ctypes.c_int64
    ms = ctypes.c_double(0.0)
    for warmup, iters in ((1, 0), (1, -3), (-1, 2)):
        assert shim.shim_moe_time(b"/nonexistent/model.bin", I(0), fptr(x), I(2), I(4), I(warmup),
                                  I(iters), ctypes.byref(ms)) == INVALID
        assert "iters" in err(shim)


# ---------------------------------------------------------------- GPU side
@pytest.mark.gpu
def test_tensor_pinned(shim):
    assert shim.shim_tensor_semantics(1) == 0, err(shim)


@pytest.mark.gpu
def test_layer_norm_bit_exact(shim, orc):
    rng = np.random.default_rng(8)
    rows, h = 45, 300
    x = (1 + 3 * rng.normal(size=(rows, h))).astype(np.float32)
    w = rng.normal(size=h).astype(np.float32)
    b = rng.normal(size=h).astype(np.float32)
    y = np.empty_like(x)
    I = ctypes.c_int64
    rc = shim.shim_layer_norm(fptr(x), I(rows), I(h), fptr(w), fptr(b), ctypes.c_float(1e-5),
                              fptr(y))
    assert rc == 0, err(shim)
    want, _, _ = orc.layer_norm(x, w, b, 1e-5, orc.CONTRACT_FMA)
    assert np.array_equal(y, want)


@pytest.mark.gpu
def test_tensor_ops_vs_oracle(shim, orc):
    rng = np.random.default_rng(1)
    m, k, n = 37, 70, 29
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    bt = rng.uniform(-1, 1, (n, k)).astype(np.float32)
    c = np.empty((m, n), np.float32)
    I = ctypes.c_int64
    assert shim.shim_matmul_transposed(fptr(a), I(m), I(k), fptr(bt), I(n), fptr(c)) == 0, err(shim)
    assert_close(c, orc.matmul_nt(a, bt), what="matmul_transposed")
    b = np.ascontiguousarray(bt.T)
    assert shim.shim_matmul(fptr(a), I(m), I(k), fptr(b), I(n), fptr(c)) == 0, err(shim)
    assert_close(c, orc.matmul_nn(a, b), what="matmul")
    x = np.linspace(-30, 30, 1001).astype(np.float32)
    u = normal(rng, (1001,))
    s = np.empty_like(x)
    p = np.empty_like(x)
    assert shim.shim_silu_mul(fptr(x), fptr(u), I(1001), fptr(s), fptr(p)) == 0, err(shim)
    assert np.array_equal(s, orc.silu(x))           # bit-exact
    assert np.array_equal(p, orc.mul(orc.silu(x), u))


@pytest.mark.gpu
def test_linear_mlp_moe_vs_oracle(shim, orc, tmp_path):
    rng = np.random.default_rng(2)
    h, ff, E, rows = 256, 192, 16, 300
    base = "model.layers.3.block_sparse_moe"
    tensors = {"proj.weight": normal(rng, (96, h), 0.02), "proj.bias": normal(rng, (96,), 0.1),
               f"{base}.gate.weight": normal(rng, (E, h), 0.02)}
    for e in range(E):
        tensors[f"{base}.experts.{e}.w1.weight"] = normal(rng, (ff, h), 0.02)
        tensors[f"{base}.experts.{e}.w3.weight"] = normal(rng, (ff, h), 0.02)
        tensors[f"{base}.experts.{e}.w2.weight"] = normal(rng, (h, ff), 0.02)
    path = str(tmp_path / "model.bin").encode()
    write_model_bin(path.decode(), tensors)
    x = normal(rng, (rows, h))
    I = ctypes.c_int64

    y = np.empty((rows, 96), np.float32)
    assert shim.shim_linear(path, b"proj.weight", b"proj.bias", fptr(x), I(rows), I(h), fptr(y),
                            I(96)) == 0, err(shim)
    assert_close(y, orc.matmul_nt(x, tensors["proj.weight"]) + tensors["proj.bias"],
                 what="Linear")

    y = np.empty((rows, h), np.float32)
    pre = f"{base}.experts.5".encode()
    assert shim.shim_mlp(path, pre, fptr(x), I(rows), I(h), fptr(y)) == 0, err(shim)
    w1 = tensors[f"{base}.experts.5.w1.weight"]
    w3 = tensors[f"{base}.experts.5.w3.weight"]
    w2 = tensors[f"{base}.experts.5.w2.weight"]
    ref = orc.matmul_nt(orc.mul(orc.silu(orc.matmul_nt(x, w1)), orc.matmul_nt(x, w3)), w2)
    assert_close(y, ref, what="PhiMLP")

    stack = lambda n: np.stack([tensors[f"{base}.experts.{e}.{n}.weight"] for e in range(E)])
    for contract in (0, 1):
        topk = np.empty((rows, 2), np.int32)
        assert shim.shim_moe(path, I(3), contract, fptr(x), I(rows), I(h), fptr(y),
                             fptr(topk)) == 0, err(shim)
        ry, ridx, _ = orc.moe_forward(x, tensors[f"{base}.gate.weight"], stack("w1"),
                                      stack("w3"), stack("w2"), 2, contract=contract)
        assert np.array_equal(topk, ridx)
        assert_close(y, ry, what=f"PhiMoE contract={contract}")
    # the host-to-host timing entry (PCIe copies included) runs the same layer
    ms = ctypes.c_double(0.0)
    assert shim.shim_moe_time(path, I(3), fptr(x), I(rows), I(h), I(1), I(2),
                              ctypes.byref(ms)) == 0, err(shim)
    assert ms.value > 0.0


def test_moe_missing_expert_raises(shim, tmp_path):
    # PhiMoE loads every expert before it uploads anything: no device needed
    rng = np.random.default_rng(3)
    base = "model.layers.0.block_sparse_moe"
    tensors = {f"{base}.gate.weight": normal(rng, (2, 8))}
    tensors[f"{base}.experts.0.w1.weight"] = normal(rng, (4, 8))
    tensors[f"{base}.experts.0.w3.weight"] = normal(rng, (4, 8))
    tensors[f"{base}.experts.0.w2.weight"] = normal(rng, (8, 4))
    path = str(tmp_path / "model.bin")
    write_model_bin(path, tensors)
    x = normal(rng, (4, 8))
    y = np.empty((4, 8), np.float32)
    topk = np.empty((4, 2), np.int32)
    I = ctypes.c_int64
    rc = shim.shim_moe(path.encode(), I(0), 1, fptr(x), I(4), I(8), fptr(y), fptr(topk))
    assert rc == RUNTIME and err(shim) == f"missing tensor: {base}.experts.1.w1.weight"


@pytest.mark.gpu
def test_add_bias_and_rope_bit_exact(shim, orc):
    rng = np.random.default_rng(6)
    I = ctypes.c_int64
    rows, cols = 33, 40
    a, b = normal(rng, (rows, cols)), normal(rng, (rows, cols))
    bias = normal(rng, (cols,))
    out = np.empty_like(a)
    assert shim.shim_add_and_bias(fptr(a), fptr(b), fptr(bias), I(rows), I(cols),
                                  fptr(out)) == 0, err(shim)
    assert np.array_equal(out, (a + b) + bias[None, :])
    # rows past seq_len stay as they are, as in the reference's loop over s < seq_len
    rows, S, H, KVH, hd = 12, 9, 4, 2, 16
    q, k = normal(rng, (rows, H * hd)), normal(rng, (rows, KVH * hd))
    gq, gk = q.copy(), k.copy()
    assert shim.shim_rope(fptr(gq), fptr(gk), I(rows), I(S), I(H), I(KVH), I(hd),
                          ctypes.c_float(10000.0)) == 0, err(shim)
    rq, rk = orc.rope(q[:S], k[:S], 1, S, H, KVH, hd)
    assert np.array_equal(gq[:S], rq) and np.array_equal(gk[:S], rk)
    assert np.array_equal(gq[S:], q[S:]) and np.array_equal(gk[S:], k[S:])


def _decoder_layer_tensors(rng, li, h, E, ff):
    """Weights of decoder layer li in the reference's names; the apss26
    attention shape: 16 query heads, 4 key heads, head_dim 128."""
    qw, kw = 16 * 128, 4 * 128
    p = f"model.layers.{li}"
    t = {f"{p}.input_layernorm.weight": 1 + normal(rng, (h,), 0.1),
         f"{p}.input_layernorm.bias": normal(rng, (h,), 0.1),
         f"{p}.post_attention_layernorm.weight": 1 + normal(rng, (h,), 0.1),
         f"{p}.post_attention_layernorm.bias": normal(rng, (h,), 0.1),
         f"{p}.block_sparse_moe.gate.weight": normal(rng, (E, h), 0.02)}
    for name, out, inp in (("q_proj", qw, h), ("k_proj", kw, h), ("v_proj", kw, h),
                           ("o_proj", h, qw)):
        t[f"{p}.self_attn.{name}.weight"] = normal(rng, (out, inp), 0.02)
        t[f"{p}.self_attn.{name}.bias"] = normal(rng, (out,), 0.02)
    for e in range(E):
        t[f"{p}.block_sparse_moe.experts.{e}.w1.weight"] = normal(rng, (ff, h), 0.02)
        t[f"{p}.block_sparse_moe.experts.{e}.w3.weight"] = normal(rng, (ff, h), 0.02)
        t[f"{p}.block_sparse_moe.experts.{e}.w2.weight"] = normal(rng, (h, ff), 0.02)
    return t


def _oracle_layer(t, li, E):
    """The names of oracle/decoder.py for the reference's layer li."""
    p = f"model.layers.{li}"
    L = {"input_norm_w": t[f"{p}.input_layernorm.weight"],
         "input_norm_b": t[f"{p}.input_layernorm.bias"],
         "post_norm_w": t[f"{p}.post_attention_layernorm.weight"],
         "post_norm_b": t[f"{p}.post_attention_layernorm.bias"],
         "gate_w": t[f"{p}.block_sparse_moe.gate.weight"]}
    for n in ("q", "k", "v", "o"):
        L[f"{n}_w"] = t[f"{p}.self_attn.{n}_proj.weight"]
        L[f"{n}_b"] = t[f"{p}.self_attn.{n}_proj.bias"]
    for n in ("w1", "w3", "w2"):
        L[n] = np.stack([t[f"{p}.block_sparse_moe.experts.{e}.{n}.weight"] for e in range(E)])
    return L


@pytest.mark.gpu
@pytest.mark.parametrize("s", [37, 64])
def test_attention_and_decoder_layer_vs_oracle(shim, orc, tmp_path, s):
    # s = 37 is not a multiple of the attention kernels' 16-row granule: the
    # drop-in pads the sequence at its end, which the causal mask leaves exact
    import types
    from oracle import decoder as od
    rng = np.random.default_rng(40 + s)
    h, E, ff, li = 256, 16, 64, 2
    t = _decoder_layer_tensors(rng, li, h, E, ff)
    path = str(tmp_path / "model.bin")
    write_model_bin(path, t)
    cfg = types.SimpleNamespace(norm="layer", norm_eps=1e-5, heads=16, kv_heads=4, head_dim=128,
                                rope_theta=10000.0, window=2047, top_k=2,
                                router=orc.ROUTER_PHI_QUANT, contract=orc.CONTRACT_FMA)
    L = _oracle_layer(t, li, E)
    x = normal(rng, (s, h))
    I = ctypes.c_int64
    y = np.empty((s, h), np.float32)
    assert shim.shim_attention(path.encode(), I(li), fptr(x), I(s), I(h), fptr(y)) == 0, err(shim)
    q, k, v = (od.linear(x, L[f"{n}_w"], L[f"{n}_b"], cfg.contract) for n in "qkv")
    q, k = orc.rope(q, k, 1, s, 16, 4, 128)
    a = orc.attention(q, k, v, 1, s, 16, 4, 128, window=2047)
    assert_close(y, od.linear(a, L["o_w"], L["o_b"], cfg.contract), what="PhiAttention")
    assert shim.shim_decoder_layer(path.encode(), I(li), fptr(x), I(s), I(h), fptr(y)) == 0, \
        err(shim)
    ref, _, _ = od.layer_forward(x, L, cfg, 1, s)
    assert_close(y, ref, what="PhiDecoderLayer")


# ------------------------------------------------------ driver formats (CPU)
def _write_inputs(path, seqs, batch=None, max_seq=None):
    with open(path, "wb") as f:
        f.write(struct.pack("<II", len(seqs) if batch is None else batch,
                            max(len(s) for s in seqs) if max_seq is None else max_seq))
        for s in seqs:
            f.write(struct.pack("<I", len(s)) + np.asarray(s, np.int32).tobytes())


def test_driver_read_inputs_and_its_errors(shim, tmp_path):
    I = ctypes.c_int64
    p = str(tmp_path / "inputs.bin")
    seqs = [[5, 6, 7], list(range(10)), [31999]]
    _write_inputs(p, seqs, max_seq=12)
    lens, ids = np.zeros(8, np.int32), np.zeros(64, np.int32)
    b, ms = I(), I()
    assert shim.shim_read_inputs(p.encode(), I(64), fptr(lens), fptr(ids), ctypes.byref(b),
                                 ctypes.byref(ms)) == 0, err(shim)
    assert b.value == 3 and ms.value == 12 and lens[:3].tolist() == [3, 10, 1]
    assert ids[:14].tolist() == sum(seqs, [])
    cases = [(dict(batch=0), "invalid input header"), (dict(max_seq=4097), "invalid input header"),
             (dict(max_seq=2), "invalid sequence length in input")]
    for kw, msg in cases:
        _write_inputs(p, seqs, **kw)
        assert shim.shim_read_inputs(p.encode(), I(64), fptr(lens), fptr(ids), ctypes.byref(b),
                                     ctypes.byref(ms)) == RUNTIME
        assert err(shim) == msg
    _write_inputs(p, [[1, 2], [3]])
    raw = open(p, "rb").read()
    open(p, "wb").write(raw[:-2])
    assert shim.shim_read_inputs(p.encode(), I(64), fptr(lens), fptr(ids), ctypes.byref(b),
                                 ctypes.byref(ms)) == RUNTIME and err(shim) == "truncated input"
    missing = str(tmp_path / "none.bin")
    assert shim.shim_read_inputs(missing.encode(), I(64), fptr(lens), fptr(ids), ctypes.byref(b),
                                 ctypes.byref(ms)) == RUNTIME
    assert err(shim) == "cannot open input: " + missing


def test_driver_outputs_and_the_validation_rule(shim, tmp_path):
    I = ctypes.c_int64
    rng = np.random.default_rng(5)
    out = normal(rng, (3, 7))
    p = str(tmp_path / "outputs.bin")
    assert shim.shim_write_outputs(p.encode(), fptr(out), I(3), I(7)) == 0, err(shim)
    raw = open(p, "rb").read()
    assert struct.unpack("<II", raw[:8]) == (3, 7)
    assert np.array_equal(np.frombuffer(raw[8:], np.float32).reshape(3, 7), out)
    ans = str(tmp_path / "answers.bin")

    def verdict(answer, output):
        answer.astype(np.float32).tofile(ans)
        ok = ctypes.c_int(-1)
        assert shim.shim_validate(ans.encode(), fptr(output), I(3), I(7), ctypes.byref(ok)) == 0
        return ok.value

    a = out.copy()
    a[1, 2] = 1.0
    assert verdict(a, a.copy()) == 1
    o = a.copy(); o[1, 2] = 1.0025  # abs 2.5e-3 <= 3e-3
    assert verdict(a, o) == 1
    o = a.copy(); o[1, 2] = 1.01  # abs and rel 1e-2
    assert verdict(a, o) == 0
    a2 = a.copy(); a2[0, 0] = 1e-9  # near zero the rule is absolute
    o = a2.copy(); o[0, 0] = 2e-3
    assert verdict(a2, o) == 1
    o[0, 0] = 1e-2
    assert verdict(a2, o) == 0
    big = a.copy(); big[2, 3] = 1000.0
    o = big.copy(); o[2, 3] = 1002.0  # abs 2 but rel 2e-3
    assert verdict(big, o) == 1
    o = a.copy(); o[2, 6] = np.nan
    assert verdict(a, o) == 0
    a[:2].tofile(ans)  # too short
    ok = ctypes.c_int(-1)
    assert shim.shim_validate(ans.encode(), fptr(out), I(3), I(7), ctypes.byref(ok)) == RUNTIME
    assert err(shim).startswith("invalid answer size: expected at least 84 bytes")


def test_driver_decode_format_and_rule(shim, tmp_path):
    I = ctypes.c_int64
    rng = np.random.default_rng(6)
    B, S, V = 2, 3, 50
    logits = normal(rng, (B, S, V))
    logits[1, 1:] = 0.0
    lens = np.array([3, 1], np.int32)
    gen = np.array([[4, 9, 2], [7, -1, -1]], np.int32)
    p = str(tmp_path / "decode.bin")
    assert shim.shim_write_decode(p.encode(), fptr(logits), fptr(lens), fptr(gen), I(B), I(S),
                                  I(V)) == 0, err(shim)
    raw = open(p, "rb").read()
    assert struct.unpack("<III", raw[:12]) == (B, S, V)
    assert np.frombuffer(raw[12:20], np.uint32).tolist() == [3, 1]
    assert np.frombuffer(raw[20:44], np.int32).reshape(B, S).tolist() == gen.tolist()
    assert np.array_equal(np.frombuffer(raw[44:], np.float32).reshape(B, S, V), logits)

    def verdict(lg, ln, gn):
        ok = ctypes.c_int(-1)
        assert shim.shim_validate_decode(p.encode(), fptr(lg), fptr(ln), fptr(gn), I(B), I(S),
                                         I(V), ctypes.byref(ok)) == 0, err(shim)
        return ok.value

    assert verdict(logits, lens, gen) == 1
    g = gen.copy(); g[0, 1] = 5
    assert verdict(logits, lens, g) == 0  # token
    ln = lens.copy(); ln[1] = 2
    g = gen.copy(); g[1, 1] = 3
    assert verdict(logits, ln, g) == 0  # length
    lg = logits.copy(); lg[0, 0, 3] += 0.05
    assert verdict(lg, lens, gen) == 0  # step 0: the prefill rule
    lg = logits.copy(); lg[0, 2] += 1e-3
    assert verdict(lg, lens, gen) == 1  # later steps: vector statistics
    lg = logits.copy(); lg[0, 2] += 0.5
    assert verdict(lg, lens, gen) == 0
    lg = logits.copy(); lg[0, 1, 0] = np.inf
    assert verdict(lg, lens, gen) == 0
    ok = ctypes.c_int(-1)
    assert shim.shim_validate_decode(p.encode(), fptr(logits), fptr(lens), fptr(gen), I(B),
                                     I(S + 1), I(V), ctypes.byref(ok)) == RUNTIME
    assert err(shim) == "decode answer header mismatch"


# ------------------------------------------------------ the model (GPU)
def _model_tensors(rng, layers, h, E, ff, vocab):
    t = {"model.embed_tokens.weight": normal(rng, (vocab, h)),
         "model.norm.weight": 1 + normal(rng, (h,), 0.1), "model.norm.bias": normal(rng, (h,), 0.1),
         "lm_head.weight": normal(rng, (vocab, h), 0.02), "lm_head.bias": normal(rng, (vocab,), 0.02)}
    for li in range(layers):
        t.update(_decoder_layer_tensors(rng, li, h, E, ff))
    return t


def _oracle_model(orc, t, layers, E):
    import types
    W = {"embed": t["model.embed_tokens.weight"], "final_norm_w": t["model.norm.weight"],
         "final_norm_b": t["model.norm.bias"], "lm_head_w": t["lm_head.weight"],
         "lm_head_b": t["lm_head.bias"], "layers": [_oracle_layer(t, li, E) for li in range(layers)]}
    cfg = types.SimpleNamespace(norm="layer", norm_eps=1e-5, heads=16, kv_heads=4, head_dim=128,
                                rope_theta=10000.0, window=2047, top_k=2,
                                router=orc.ROUTER_PHI_QUANT, contract=orc.CONTRACT_FMA, layers=layers)
    return W, cfg


@pytest.mark.gpu
def test_model_generate_and_decode_vs_oracle(shim, orc, tmp_path):
    # a batch with shared prefixes, a duplicate and a sequence that is a
    # prefix of another: the trie computes each prefix once; every sequence's
    # logits must equal the oracle's run of that sequence alone
    from oracle import decoder as od
    rng = np.random.default_rng(50)
    L, h, E, ff, V = 2, 256, 4, 64, 32064
    t = _model_tensors(rng, L, h, E, ff, V)
    path = str(tmp_path / "model.bin")
    write_model_bin(path, t)
    W, cfg = _oracle_model(orc, t, L, E)
    base = rng.integers(0, 32000, 24)
    seqs = [base[:24], base[:9], np.concatenate([base[:9], [11, 12]]), base[:24],
            rng.integers(0, 32000, 17), base[:1]]
    lens = np.array([len(s) for s in seqs], np.int32)
    ids = np.concatenate(seqs).astype(np.int32)
    I = ctypes.c_int64
    got = np.empty((len(seqs), V), np.float32)
    assert shim.shim_model_generate(path.encode(), fptr(lens), fptr(ids), I(len(seqs)), fptr(got),
                                    I(V)) == 0, err(shim)
    for b, s in enumerate(seqs):
        ref, _, _ = od.generate(np.asarray(s)[None, :], W, cfg)
        assert_close(got[b], ref[0], what=f"sequence {b}")
    # greedy decode of 3 tokens: the oracle's loop over each sequence alone
    steps = 3
    dl = np.empty((len(seqs), steps, V), np.float32)
    gl = np.empty(len(seqs), np.int32)
    gi = np.empty((len(seqs), steps), np.int32)
    assert shim.shim_model_decode(path.encode(), fptr(lens), fptr(ids), I(len(seqs)), I(steps),
                                  fptr(dl), fptr(gl), fptr(gi)) == 0, err(shim)
    for b, s in enumerate(seqs[:4]):
        prefix = list(s)
        for st in range(steps):
            ref, _, _ = od.generate(np.asarray(prefix)[None, :], W, cfg)
            nxt = int(np.argmax(ref[0]))
            assert gi[b, st] == nxt, f"sequence {b} step {st}"
            assert_close(dl[b, st], ref[0], what=f"decode logits {b},{st}")
            prefix.append(nxt)
        assert gl[b] == steps


@pytest.mark.gpu
def test_model_generate_repeated_tokens_vs_oracle(shim, orc, tmp_path):
    # tokens from a pool of 7, so most trie nodes share their token with
    # nodes at other depths and in other branches: the first layer's norm
    # and q/k/v run over the 7 distinct tokens' rows and are expanded to the
    # nodes (RoPE at each node's own depth); every sequence's logits must
    # still equal the oracle's run of that sequence alone.  A second batch
    # without repeats takes the all-nodes path on the same model.
    from oracle import decoder as od
    rng = np.random.default_rng(52)
    L, h, E, ff, V = 3, 256, 4, 64, 32064
    t = _model_tensors(rng, L, h, E, ff, V)
    path = str(tmp_path / "model.bin")
    write_model_bin(path, t)
    W, cfg = _oracle_model(orc, t, L, E)
    pool = rng.integers(0, 32000, 7)
    base = pool[rng.integers(0, 7, 20)]
    seqs = [base, base[:6], np.concatenate([base[:6], pool[[3, 3, 0]]]), pool[rng.integers(0, 7, 13)],
            np.full(9, pool[2]), pool[rng.integers(0, 7, 1)]]
    distinct = [rng.permutation(32000)[:n] for n in (11, 5, 17)]
    for batch in (seqs, distinct):
        lens = np.array([len(s) for s in batch], np.int32)
        ids = np.concatenate(batch).astype(np.int32)
        got = np.empty((len(batch), V), np.float32)
        assert shim.shim_model_generate(path.encode(), fptr(lens), fptr(ids), ctypes.c_int64(len(batch)),
                                        fptr(got), ctypes.c_int64(V)) == 0, err(shim)
        for b, sq in enumerate(batch):
            ref, _, _ = od.generate(np.asarray(sq)[None, :], W, cfg)
            assert_close(got[b], ref[0], what=f"sequence {b}")


@pytest.mark.gpu
def test_model_decode_stops_at_eos_and_rejects_bad_input(shim, orc, tmp_path):
    rng = np.random.default_rng(51)
    L, h, E, ff, V = 1, 256, 4, 64, 32064
    t = _model_tensors(rng, L, h, E, ff, V)
    t["lm_head.bias"][32000] = 100.0  # EOS wins every step
    path = str(tmp_path / "model.bin")
    write_model_bin(path, t)
    I = ctypes.c_int64
    lens = np.array([5, 3], np.int32)
    ids = rng.integers(0, 32000, 8).astype(np.int32)
    dl = np.full((2, 4, V), 7.0, np.float32)
    gl = np.empty(2, np.int32)
    gi = np.empty((2, 4), np.int32)
    assert shim.shim_model_decode(path.encode(), fptr(lens), fptr(ids), I(2), I(4), fptr(dl),
                                  fptr(gl), fptr(gi)) == 0, err(shim)
    assert gl.tolist() == [1, 1] and gi[:, 0].tolist() == [32000, 32000]
    assert np.all(gi[:, 1:] == -1) and np.all(dl[:, 1:] == 0.0) and np.all(dl[:, 0] != 0.0)
    want = {1: (RUNTIME, "generate received an empty input batch"), 2: (INVALID, "empty input"),
            3: (INVALID, "token out of vocabulary"), 4: (INVALID, "sequence is too long")}
    for which, (code, msg) in want.items():
        assert shim.shim_model_bad_input(path.encode(), which) == code, which
        assert err(shim) == msg
