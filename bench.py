"""Benchmark of the MoE layer forward on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config c3|c4|c5|ref] [--block]
                    [--cpu-seconds S] [--no-extra]
    python bench.py --sgemm        (config 2: the SGEMM sweep, a line per shape)
    python bench.py --decoder      (config 5: the whole 4-layer decoder prefill)
    python bench.py --dropin       (the C++ drop-in PhiMoE::forward, host tensors,
                                    at the reference's layer shape)
    python bench.py --model        (the C++ drop-in PhiTinyMoEModel::generate on the
                                    reference's model shape and batch)

A step is one moe_layer_forward (gate -> route -> permute -> grouped expert
FFN -> combine) over one batch of synthetic tokens whose inputs and weights
are already resident in HBM.  The default workload is config 3 of the
baseline: the Mixtral-shaped fp32 layer, 4096 tokens x d_model 4096, 8
experts top-2, SwiGLU d_ff 14336, weights N(0, 0.02), inputs N(0, 1),
softmax over the selected logits.

Prints ONE JSON line: tokens/s of the whole layer, the roofline of the
dominant kernel (the grouped w1/w3 SwiGLU GEMM, fp32 MFMA bound) measured
with HIP events on the stream the kernels run on, and the CPU path (the
oracle restatement of the reference's PhiMoE::forward) timed on a bounded
token sample on this host's cores.  The default run (config 3) then times
the other layer shapes (config 5's MoE FFN, the reference's own layer,
config 4) the same way, without CPU legs, under `other_layer_shapes`.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
METRIC = "MoE layer tokens/sec + expert-GEMM TFLOP/s (% fp32 MFMA peak), 1 MI355X"
FP32_MFMA_PEAK_TFLOPS = 157.3
HBM_PEAK_GBS = 8000.0
NORM_EPS = 1e-5
SPINUP_S = 1.0

CONFIGS = {
    # name: T, d, E, k, d_ff, router bias (Zipf s) or None
    "c3": dict(T=4096, d=4096, E=8, k=2, d_ff=14336, zipf=None, norm="layer",
               workload="mixtral_moe_layer_fp32"),
    "c4": dict(T=16384, d=2048, E=64, k=8, d_ff=1408, zipf=1.2, norm="layer",
               workload="fine_grained_zipf_moe_layer_fp32"),
    # the MoE FFN of config 5's decoder (batch 8 x seq 512 tokens, d 1024)
    "c5": dict(T=4096, d=1024, E=8, k=2, d_ff=2816, zipf=None, norm="rms",
               workload="decoder_prefill_moe_ffn_fp32"),
    # the reference's own MoE layer (Phi-tiny-MoE: d 4096, 16 experts of d_ff 448,
    # its quantised top-2 router) at its contest input's 15,583 rows, the shape its
    # per-layer expert GEMM times are quoted on (docs/lab-note.md:4294-4296)
    "ref": dict(T=15583, d=4096, E=16, k=2, d_ff=448, zipf=None, norm="layer",
                workload="phi_tiny_moe_layer_fp32", router="phi_quant"),
}
# The reference's grouped expert GEMM times per layer on its RTX 3090 (summed
# over 32 layers in docs/lab-note.md:4294-4296: w13 363 ms, w2 191 ms), for
# the "ref" workload only.
REF_GEMM_MS = {"expert_w13_swiglu": 363.0 / 32, "expert_w2": 191.0 / 32}

# Config 2: standalone SGEMM sweep (NN, row-major, A and B ~ U[-1, 1]).
SGEMM_SHAPES = [(1024, 1024, 1024), (2048, 2048, 2048), (4096, 4096, 4096), (8192, 8192, 8192),
                (16, 14336, 4096), (64, 14336, 4096), (256, 14336, 4096), (512, 14336, 4096)]


def sgemm_sweep(args):
    """One JSON line per config-2 shape: TFLOP/s against the fp32 MFMA peak
    and the HBM roofline (max of flop time and byte time).  Each shape runs
    untimed for a while first (SPINUP_S before the first shape, a fifth of
    it before the others) so that every line is measured at the clock a
    loaded GPU holds, as the layer bench is; the warm-up calls follow."""
    import torch
    pkg = load_pkg()
    ctx = pkg.Context(0)
    g = torch.Generator(device="cuda").manual_seed(0)
    first = True
    for layout in ("nn", "nt"):
        for M, N, K in SGEMM_SHAPES:
            a = torch.rand((M, K), device="cuda", generator=g) * 2 - 1
            b = (torch.rand((K, N), device="cuda", generator=g) * 2 - 1) if layout == "nn" else \
                (torch.rand((N, K), device="cuda", generator=g) * 2 - 1)
            c = torch.empty((M, N), device="cuda")
            fn = ctx.sgemm_nn if layout == "nn" else ctx.sgemm_nt
            spin = SPINUP_S if first else SPINUP_S / 5
            first = False
            t_spin = time.perf_counter()
            while time.perf_counter() - t_spin < spin:
                for _ in range(4):
                    fn(a, b, c)
                torch.cuda.synchronize()
            for _ in range(args.warmup):
                fn(a, b, c)
            ctx.reset_timing()
            ctx.set_timing(True)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(args.steps):
                fn(a, b, c)
            torch.cuda.synchronize()
            wall = (time.perf_counter() - t0) / args.steps
            ctx.set_timing(False)
            ms, n = ctx.kernel_times()[f"sgemm_{layout}"]
            t = ms / n * 1e-3
            flops = 2.0 * M * N * K
            nbytes = 4.0 * (M * K + K * N + M * N)
            floor = max(flops / (FP32_MFMA_PEAK_TFLOPS * 1e12), nbytes / (HBM_PEAK_GBS * 1e9))
            print(json.dumps({"workload": "sgemm", "layout": layout, "M": M, "N": N, "K": K,
                              "kernel_ms": t * 1e3, "wall_ms": wall * 1e3,
                              "tflops": flops / t / 1e12,
                              "frac_fp32_mfma_peak": flops / t / 1e12 / FP32_MFMA_PEAK_TFLOPS,
                              "frac_of_roofline_time": floor / t}), flush=True)
            del a, b, c
    ctx.close()


def load_pkg():
    pkg_dir = os.path.join(ROOT, "accelerating-moe-inference_amd")
    spec = importlib.util.spec_from_file_location(
        "moe_amd", os.path.join(pkg_dir, "__init__.py"), submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["moe_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def zipf_bias(E, s):
    import numpy as np
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    p /= p.sum()
    return np.log(p).astype(np.float32)


def hbm_kernel_rates(avg, T, d, E, k, block, w2_splits):
    """Achieved HBM rate of the routing, permutation, combine and norm kernels
    against the 8 TB/s peak: algorithmic bytes (each operand read once, each
    result written once) over the kernel's HIP-event time.  The combine reads
    the w2_splits K-split partial row buffers the layer's w2 wrote."""
    nb = -(-T // 256)
    pairs = T * k
    algo = {
        "gate_logits": 4 * (T * d + E * d + T * E),
        "route_softmax": 4 * (T * E + E) + 8 * pairs,
        "route_phi": 4 * (T * E + E) + 8 * pairs,
        "perm_count": 4 * pairs + 4 * E * nb,
        "perm_scan": 8 * E * nb + 4 * (E + 1),
        "perm_place": 4 * pairs + 4 * E * nb + 8 * pairs,
        "layer_norm": 8 * T * d + 8 * T,
        "rms_norm": 8 * T * d + 4 * T,
    }
    out = {}
    for name, b in algo.items():
        if name in avg:
            gbs = b / (avg[name] * 1e-3) / 1e9
            out[name] = {"bytes": b, "ms": round(avg[name], 5), "GB/s": round(gbs, 1),
                         "frac": round(gbs / HBM_PEAK_GBS, 4)}
    if "combine" in avg:
        S = w2_splits
        b = 4 * S * pairs * d + 12 * pairs + 4 * T * d * (2 if block else 1)
        gbs = b / (avg["combine"] * 1e-3) / 1e9
        out["combine"] = {"bytes": b, "ms": round(avg["combine"], 5), "GB/s": round(gbs, 1),
                          "frac": round(gbs / HBM_PEAK_GBS, 4), "w2_splits": S}
    return out


def host_cpu():
    """The host's CPU model and logical core count (the CPU baseline's hardware)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return f"{model}, {os.cpu_count()} logical cores on the host"


def tile_cover_sample(gidx, E, bm=128, block=32):
    """Tokens whose packed rows land in every bm-row m-tile of every expert of
    the grouped GEMMs (per tile its last row, so each expert's ragged last
    tile, and one row of a further 32-row MFMA block), then every other token
    in ascending order.  Routing is per token, so the layer recomputed on any
    subset gives exactly those rows of the full layer."""
    import numpy as np
    T, k = gidx.shape
    order = np.argsort(gidx.ravel(), kind="stable")
    tok = order // k
    offsets = np.concatenate([[0], np.cumsum(np.bincount(gidx.ravel(), minlength=E))])
    pick = {0, T - 1}
    for e in range(E):
        n = int(offsets[e + 1] - offsets[e])
        for j in range((n + bm - 1) // bm):
            base, rows = int(offsets[e]) + j * bm, min(bm, n - j * bm)
            pick.add(int(tok[base + rows - 1]))
            lo = ((j + e) % ((rows + block - 1) // block)) * block
            pick.add(int(tok[base + lo + (j * 7 + e * 13) % min(block, rows - lo)]))
    cover = np.array(sorted(pick), dtype=np.int64)
    rest = np.setdiff1d(np.arange(T), cover)
    return np.concatenate([cover, rest]), len(cover)


def cpu_baseline(x, weights, cfg, pkg_outputs, target_s):
    """The oracle's PhiMoE::forward restatement on a token sample sized to
    about target_s seconds of CPU work (at least the tokens that cover every
    m-tile of every expert), checked against the GPU's rows; and the oracle's
    gate and router on every token, checked against the GPU's routing.  Test
    infrastructure: timed here as the reported CPU baseline, never part of
    the GPU measurement."""
    import numpy as np
    sys.path.insert(0, ROOT)
    import oracle

    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or min(16, os.cpu_count() or 1)
    oracle.set_threads(threads)
    gw, w1, w3, w2, bias = (weights[n] for n in ("gate_w", "w1", "w3", "w2", "expert_bias"))
    nw, nb = weights.get("norm_w"), weights.get("norm_b")
    k = cfg["k"]
    router = (oracle.ROUTER_PHI_QUANT if cfg.get("router") == "phi_quant"
              else oracle.ROUTER_SOFTMAX_TOPK)
    gy, gidx = pkg_outputs

    def normed(xs):
        if nw is None:
            return xs
        if nb is None:
            return oracle.rms_norm(xs, nw, NORM_EPS, oracle.CONTRACT_FMA)[0]
        return oracle.layer_norm(xs, nw, nb, NORM_EPS, oracle.CONTRACT_FMA)[0]

    def run(toks):
        t0 = time.perf_counter()
        y, idx, w = oracle.moe_forward(normed(x[toks]), gw, w1, w3, w2, k,
                                       act=oracle.ACT_SWIGLU, router_mode=router,
                                       expert_bias=bias)
        if nw is not None:  # the decoder block: y = x + MoE(norm(x))
            y = y + x[toks]
        return time.perf_counter() - t0, y, idx

    order, n_cover = tile_cover_sample(gidx, cfg["E"])
    # Grow the sample until it takes about target_s: small samples leave
    # most of the threads idle (the reference parallelises over an expert's
    # rows), so the per-token time only settles once experts hold >= threads
    # rows each.
    n = max(16, n_cover)
    while True:
        toks = np.sort(order[:n])
        dt, y, idx = run(toks)
        if dt >= 0.5 * target_s or n >= cfg["T"]:
            break
        n = int(min(cfg["T"], max(2 * n, round(0.9 * n * target_s / max(dt, 1e-9)))))
    ref_scale = float(np.max(np.abs(y))) or 1.0
    all_idx, _ = oracle.route(oracle.matmul_nt(normed(x), gw, oracle.CONTRACT_FMA), k,
                              mode=router, expert_bias=bias)
    parity = {
        "tokens": n,
        "tile_covering_tokens": n_cover,
        "routing_bit_exact": bool(np.array_equal(gidx[toks], idx)),
        "routing_bit_exact_all_tokens": bool(np.array_equal(gidx, all_idx)),
        "max_rel_err": float(np.max(np.abs(gy[toks] - y)) / ref_scale),
    }
    return {
        "value": n / dt,
        "unit": "tokens/s",
        "cores": oracle.get_threads(),
        "kind": "port",
        "host": host_cpu(),
        "sample": (f"{n} of {cfg['T']} tokens of the same layer (same weights; routing is "
                   f"per token): the {n_cover} whose packed rows cover every 128-row m-tile "
                   f"of every expert, then the lowest-numbered others; {dt:.1f} s on "
                   f"{oracle.get_threads()} threads"),
    }, parity


def decoder_cpu_baseline(tokens, W, cfg, gpu_hidden, target_s):
    """The oracle decoder (oracle/decoder.py) on a sample of the batch sized
    to about target_s seconds of CPU work: a prefix of sequence 0 while one
    sequence is more than enough, else the first m whole sequences.
    Attention is causal and sequences are independent, so the sample's rows
    are exactly those rows of the full prefill."""
    import numpy as np
    sys.path.insert(0, ROOT)
    import oracle
    from oracle import decoder as od

    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or min(16, os.cpu_count() or 1)
    oracle.set_threads(threads)
    B, S = tokens.shape
    m, n = 1, 16
    while True:
        t0 = time.perf_counter()
        _, x, _ = od.generate(tokens[:m, :n], W, cfg)
        dt = time.perf_counter() - t0
        if dt >= 0.5 * target_s or m >= B:
            break
        if n < S:
            n = int(min(S, max(2 * n, 16 * round(0.9 * n * target_s / max(dt, 1e-9) / 16))))
        else:
            m = int(min(B, max(m + 1, round(0.9 * m * target_s / max(dt, 1e-9)))))
    ref = gpu_hidden.reshape(B, S, -1)[:m, :n].reshape(m * n, -1)
    parity = {"tokens": m * n,
              "hidden_max_rel_err": float(np.max(np.abs(ref - x)) / (np.max(np.abs(x)) or 1.0))}
    what = (f"first {n} positions of sequence 0" if m == 1 and n < S
            else f"the first {m} whole sequences")
    return {
        "value": m * n / dt,
        "unit": "tokens/s",
        "cores": oracle.get_threads(),
        "kind": "port",
        "host": host_cpu(),
        "sample": (f"{what} of {B} x {S} (all {cfg.layers} layers, same weights; causal "
                   f"attention, so these rows are those of the full prefill), {dt:.1f} s on "
                   f"{oracle.get_threads()} threads"),
    }, parity


def write_model_bin(path, tensors):
    """The reference's model.bin layout (src/model_loader.cu:14-30): u32 count;
    per tensor u32 name length, name, u32 ndim, u32 dims, u64 offset, u64
    bytes; the fp32 data at the offsets."""
    import struct
    import numpy as np
    header = 4 + sum(4 + len(n.encode()) + 4 + 4 * a.ndim + 16 for n, a in tensors.items())
    blob = bytearray(struct.pack("<I", len(tensors)))
    off = header
    for name, a in tensors.items():
        nb = name.encode()
        blob += struct.pack("<I", len(nb)) + nb + struct.pack("<I", a.ndim)
        blob += struct.pack(f"<{a.ndim}I", *a.shape) + struct.pack("<QQ", off, a.nbytes)
        off += a.nbytes
    with open(path, "wb") as f:
        f.write(bytes(blob))
        for a in tensors.values():
            f.write(np.ascontiguousarray(a, dtype=np.float32).tobytes())


def dropin_bench(args):
    """The C++ drop-in's PhiMoE::forward (host Tensors in and out, so the PCIe
    copies are inside the time) at the reference's layer shape, through the
    C shim the drop-in tests use (tests/cpp/libdropin_shim.so): weights in a
    model.bin of the reference's format, 15,583 rows of d 4096."""
    import ctypes
    import tempfile
    import numpy as np
    cfg = CONFIGS["ref"]
    T, d, E, d_ff = cfg["T"], cfg["d"], cfg["E"], cfg["d_ff"]
    rng = np.random.default_rng(0)
    base = "model.layers.0.block_sparse_moe"
    tensors = {f"{base}.gate.weight": (0.02 * rng.standard_normal((E, d))).astype(np.float32)}
    for e in range(E):
        for name, shape in (("w1", (d_ff, d)), ("w2", (d, d_ff)), ("w3", (d_ff, d))):
            tensors[f"{base}.experts.{e}.{name}.weight"] = (
                0.02 * rng.standard_normal(shape)).astype(np.float32)
    x = rng.standard_normal((T, d)).astype(np.float32)
    shim = ctypes.CDLL(os.path.join(ROOT, "tests", "cpp", "libdropin_shim.so"))
    shim.shim_error.restype = ctypes.c_char_p
    I = ctypes.c_int64
    ms = ctypes.c_double(0.0)
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "model.bin")
        write_model_bin(path, tensors)
        rc = shim.shim_moe_time(path.encode(), I(0), x.ctypes.data_as(ctypes.c_void_p), I(T),
                                I(d), I(args.warmup), I(args.steps), ctypes.byref(ms))
    if rc != 0:
        raise RuntimeError(f"shim_moe_time: {shim.shim_error().decode()}")
    print(json.dumps({
        "metric": "drop-in PhiMoE::forward tokens/sec, host tensors in and out (PCIe-inclusive), "
                  "1 MI355X",
        "value": T / (ms.value * 1e-3), "unit": "tokens/s", "ms_per_call": ms.value,
        "steps": args.steps, "warmup": args.warmup, "dtype": "f32",
        "data": "synthetic (seeded: x ~ N(0,1), weights ~ N(0,0.02))",
        "config": {"workload": cfg["workload"], "tokens": T, "d_model": d, "experts": E,
                   "top_k": cfg["k"], "d_ff": d_ff,
                   "router": "quantised top-2, weights 1/2 (PhiMoE::route)",
                   "io": "pageable host Tensors through the drop-in's pinned staging"},
    }))


def model_bench(args):
    """The C++ drop-in's PhiTinyMoEModel::generate (the reference's timed
    end-to-end call, src/main.cpp:584-601) on the reference's model shape
    (Phi-tiny-MoE: 32 layers, d 4096, 16 query / 4 key heads of 128, 16
    experts of d_ff 448, vocabulary 32064; random weights) over a batch
    shaped like the reference's contest input: 1024 sequences, 10-29 tokens
    each, whose first 4 tokens come from 64 shared prefixes, so the prefix
    trie removes about a fifth of the rows (the reference's input: 19,803
    tokens, 15,583 trie rows).  Host token lists in, host logits out."""
    import ctypes
    import struct
    import tempfile
    import numpy as np
    L_, h, E, ff, vocab, qw, kw = 32, 4096, 16, 448, 32064, 16 * 128, 4 * 128
    specs = [("model.embed_tokens.weight", (vocab, h), 1.0, 0.0),
             ("model.norm.weight", (h,), 0.1, 1.0), ("model.norm.bias", (h,), 0.1, 0.0),
             ("lm_head.weight", (vocab, h), 0.02, 0.0), ("lm_head.bias", (vocab,), 0.02, 0.0)]
    for li in range(L_):
        p = f"model.layers.{li}"
        specs += [(f"{p}.input_layernorm.weight", (h,), 0.1, 1.0),
                  (f"{p}.input_layernorm.bias", (h,), 0.1, 0.0),
                  (f"{p}.post_attention_layernorm.weight", (h,), 0.1, 1.0),
                  (f"{p}.post_attention_layernorm.bias", (h,), 0.1, 0.0),
                  (f"{p}.block_sparse_moe.gate.weight", (E, h), 0.02, 0.0)]
        for name, out, inp in (("q_proj", qw, h), ("k_proj", kw, h), ("v_proj", kw, h),
                               ("o_proj", h, qw)):
            specs += [(f"{p}.self_attn.{name}.weight", (out, inp), 0.02, 0.0),
                      (f"{p}.self_attn.{name}.bias", (out,), 0.02, 0.0)]
        for e in range(E):
            specs += [(f"{p}.block_sparse_moe.experts.{e}.w1.weight", (ff, h), 0.02, 0.0),
                      (f"{p}.block_sparse_moe.experts.{e}.w3.weight", (ff, h), 0.02, 0.0),
                      (f"{p}.block_sparse_moe.experts.{e}.w2.weight", (h, ff), 0.02, 0.0)]
    # every tensor is a window of one seeded N(0,1) pool (64 MiB), at its own
    # offset, scaled and shifted; each gate gets its own fresh draws
    rng = np.random.default_rng(0)
    pool = rng.standard_normal(1 << 24).astype(np.float32)
    sizes = [int(np.prod(shape)) for _, shape, _, _ in specs]
    header = 4 + sum(4 + len(n.encode()) + 4 + 4 * len(shape) + 16 for n, shape, _, _ in specs)
    # the batch: 1024 sequences, lengths 10..29, the first 4 tokens from one
    # of 64 shared prefixes
    tr = np.random.default_rng(1)
    prefixes = tr.integers(0, 32000, (64, 4))
    lens = tr.integers(10, 30, 1024).astype(np.int32)
    seqs = [np.concatenate([prefixes[tr.integers(0, 64)], tr.integers(0, 32000, n - 4)])
            for n in lens]
    nodes = len({tuple(sq[:i + 1]) for sq in seqs for i in range(len(sq))})
    ids = np.concatenate(seqs).astype(np.int32)
    shim = ctypes.CDLL(os.path.join(ROOT, "tests", "cpp", "libdropin_shim.so"))
    shim.shim_error.restype = ctypes.c_char_p
    I, D = ctypes.c_int64, ctypes.c_double
    load_s, ms = D(0.0), D(0.0)
    t0 = time.perf_counter()
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "model.bin")
        with open(path, "wb") as f:
            blob = bytearray(struct.pack("<I", len(specs)))
            off = header
            for (name, shape, _, _), n in zip(specs, sizes):
                nb = name.encode()
                blob += struct.pack("<I", len(nb)) + nb + struct.pack("<I", len(shape))
                blob += struct.pack(f"<{len(shape)}I", *shape) + struct.pack("<QQ", off, 4 * n)
                off += 4 * n
            f.write(bytes(blob))
            for i, ((name, shape, scale, shift), n) in enumerate(zip(specs, sizes)):
                if ".gate." in name:
                    a = rng.standard_normal(n).astype(np.float32)
                else:
                    a = np.resize(np.roll(pool, -((i * 7919 * 4096) % pool.size)), n)
                (a * np.float32(scale) + np.float32(shift)).astype(np.float32).tofile(f)
        write_s = time.perf_counter() - t0
        print(f"model.bin written ({off / 2**30:.1f} GiB, {write_s:.0f} s); timing generate()",
              file=sys.stderr, flush=True)
        # at least SPINUP_S of untimed calls (a call takes about 0.3 s), so the
        # timed calls run at the clock a loaded GPU holds
        warm = max(args.warmup, int(math.ceil(SPINUP_S / 0.25)))
        rc = shim.shim_model_time(path.encode(), lens.ctypes.data_as(ctypes.c_void_p),
                                  ids.ctypes.data_as(ctypes.c_void_p), I(len(lens)),
                                  I(warm), I(args.steps), ctypes.byref(load_s),
                                  ctypes.byref(ms))
    if rc != 0:
        raise RuntimeError(f"shim_model_time: {shim.shim_error().decode()}")
    seq_s = len(lens) / (ms.value * 1e-3)
    print(json.dumps({
        "metric": "drop-in PhiTinyMoEModel::generate sequences/sec (prefill, logits of the last "
                  "position), 1 MI355X",
        "value": seq_s, "unit": "seq/s", "ms_per_call": ms.value, "steps": args.steps,
        "warmup": warm, "dtype": "f32",
        "data": "synthetic (seeded random weights; random token ids with 64 shared prefixes)",
        "config": {"workload": "phi_tiny_moe_generate_fp32", "sequences": int(len(lens)),
                   "tokens": int(lens.sum()), "trie_rows": nodes, "layers": L_, "d_model": h,
                   "experts": E, "top_k": 2, "d_ff": ff, "vocab": vocab,
                   "router": "quantised top-2, weights 1/2 (PhiMoE::route)"},
        "reference_gpu_seq_s": 687.8,
        "reference_note": "the reference's end-to-end figure on one RTX 3090, 1024 sequences / "
                          "19,803 tokens of its contest input (docs/report/report.html:96)",
        "model_load_s": load_s.value,
    }))


def decoder_bench(args, pkg):
    """Config 5 as a whole: the 4-layer decoder prefill of 8 x 512 tokens
    (embedding, per layer RMS norm, q/k/v projections, RoPE, causal
    attention, o projection + residual, the MoE block with its norm and
    residual; final norm and lm_head on the last row of every sequence)."""
    import numpy as np
    import torch

    B, S = 8, 512
    cfg = pkg.DecoderConfig()
    dev = torch.device("cuda:0")
    W = pkg.random_weights(cfg, dev, seed=0)
    g = torch.Generator(device="cpu").manual_seed(1)
    tokens = torch.randint(0, cfg.vocab, (B, S), generator=g, dtype=torch.int32).to(dev)
    ctx = pkg.Context(0)
    model = pkg.DecoderModel(ctx, cfg, W)
    model.reserve(B, S)
    logits = torch.empty((B, cfg.vocab), device=dev)
    # spin-up: prefills for at least SPINUP_S, so every timed step runs at the
    # clock a loaded GPU holds; then the warm-up steps
    t_spin = time.perf_counter()
    while time.perf_counter() - t_spin < SPINUP_S:
        model.generate(tokens, logits)
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        model.generate(tokens, logits)
    torch.cuda.synchronize()
    # per-kernel HIP events over K eager steps (the breakdown and the roofline)
    ctx.reset_timing()
    ctx.set_timing(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        model.generate(tokens, logits)
    torch.cuda.synchronize()
    eager_s = time.perf_counter() - t0
    ctx.set_timing(False)
    kt = ctx.kernel_times()
    elapsed = eager_s
    graph_note = None
    if not args.no_graph:
        # the timed steps: the same prefill captured once in a HIP graph and
        # replayed (one host launch per step instead of ~70)
        from moe_amd.decoder import CapturedPrefill
        cap = CapturedPrefill(model, B, S, warmup=args.warmup)
        cap.tokens.copy_(tokens)
        for _ in range(args.warmup):
            cap.replay()
        torch.cuda.synchronize()
        check = cap.replay().clone()
        model.generate(tokens, logits)
        torch.cuda.synchronize()
        assert torch.equal(check, logits), "graph replay differs from the eager prefill"
        t0 = time.perf_counter()
        for _ in range(args.steps):
            cap.replay()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        cap.close()
        graph_note = (f"timed steps are HIP-graph replays of the prefill; the per-kernel times "
                      f"come from HIP events over {args.steps} eager steps "
                      f"({1e3 * eager_s / args.steps:.3f} ms per eager step)")
    T = B * S
    per_step = {n: ms / args.steps for n, (ms, _) in kt.items()}
    avg = {n: ms / c for n, (ms, c) in kt.items()}
    pairs = T * cfg.top_k
    # w13 launches differ in size (the pruned last layer has B*k pairs), so
    # the roofline is the step's w13 FLOPs over the step's w13 time
    full = cfg.layers - 1 if model.prune_last else cfg.layers
    tail_pairs = B * cfg.top_k if model.prune_last else 0
    flops_w13 = 2.0 * (full * pairs + tail_pairs) * cfg.d * cfg.d_ff * 2
    w13_tflops = flops_w13 / (per_step["expert_w13_swiglu"] * 1e-3) / 1e12
    qw, kw = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    tail_rows = B if model.prune_last else 0
    proj_flops = (2.0 * full * T * cfg.d * (qw + 2 * kw + qw) + 2.0 * tail_rows * cfg.d * (qw + qw)
                  + 2.0 * (cfg.layers - full) * T * cfg.d * 2 * kw + 2.0 * B * cfg.d * cfg.vocab)
    # causal attention: S(S+1)/2 (query, key) pairs per sequence and head, 2 products;
    # the pruned layer's last rows see S keys each
    attn_flops = (full * B * cfg.heads * 2 * (2.0 * cfg.head_dim * S * (S + 1) / 2)
                  + tail_rows * cfg.heads * 2 * (2.0 * cfg.head_dim * S))
    moe_flops = 2.0 * (full * pairs + tail_pairs) * cfg.d * cfg.d_ff * 3
    cpu = parity = None
    if args.cpu_seconds > 0:
        hidden = model.hidden(tokens).cpu().numpy()
        Wh = {k: (None if v is None else v.cpu().numpy()) for k, v in W.items() if k != "layers"}
        Wh["layers"] = [{k: (None if v is None else v.cpu().numpy()) for k, v in L.items()}
                        for L in W["layers"]]
        cpu, parity = decoder_cpu_baseline(tokens.cpu().numpy(), Wh, cfg, hidden,
                                           args.cpu_seconds)
    ms_per_step = 1e3 * elapsed / args.steps
    out = {
        "metric": "decoder prefill tokens/sec (config 5), 1 MI355X",
        "value": T * args.steps / elapsed,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": ("synthetic (seeded: token ids uniform over the vocabulary, embedding "
                 "N(0,1), weights N(0,0.02), norm weights 1 + N(0,0.1))"),
        "config": {"workload": "decoder_prefill_fp32", "batch": B, "seq_len": S,
                   "layers": cfg.layers, "d_model": cfg.d, "heads": cfg.heads,
                   "kv_heads": cfg.kv_heads, "experts": cfg.experts, "top_k": cfg.top_k,
                   "d_ff": cfg.d_ff, "vocab": cfg.vocab, "norm": "rms", "rope_theta":
                   cfg.rope_theta, "router": "softmax over selected top-k",
                   "lm_head": "last position of each sequence"},
        "model_tflops": (proj_flops + attn_flops + moe_flops) / (ms_per_step * 1e-3) / 1e12,
        "roofline": {
            "kernel": "expert_w13_swiglu",
            "bound": "mfma",
            "achieved": w13_tflops,
            "peak": FP32_MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": w13_tflops / FP32_MFMA_PEAK_TFLOPS,
            "traffic": None,
            "flops_per_step": flops_w13,
            "launches_per_step": cfg.layers,
            "note": (f"achieved = the step's w13 FLOPs ({full} layers x {pairs} pairs + "
                     f"{tail_pairs} pairs of the pruned layer) over the step's w13 HIP-event time"),
        },
        "kernel_ms_per_step": {n: round(v, 4) for n, v in sorted(per_step.items())},
        "kernel_avg_ms": {n: round(v, 5) for n, v in sorted(avg.items())},
        "cpu_baseline": cpu,
        "cpu_sample_parity": parity,
        "timing": graph_note or "timed steps are eager, with HIP events around every kernel",
        "eager_ms_per_step": 1e3 * eager_s / args.steps,
    }
    ctx.close()
    print(json.dumps(out))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c3", choices=sorted(CONFIGS))
    ap.add_argument("--tokens", type=int, default=None,
                    help="tokens of the layer forward (default: the configuration's)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="target CPU time of the cpu_baseline sample (0 = skip)")
    ap.add_argument("--sgemm", action="store_true",
                    help="config-2 SGEMM sweep instead of the layer (one JSON line per shape)")
    ap.add_argument("--block", action="store_true",
                    help="the layer as the decoder's MoE block: y = x + MoE(layer_norm(x))")
    ap.add_argument("--decoder", action="store_true",
                    help="config 5's whole decoder prefill (8 x 512 tokens, 4 layers)")
    ap.add_argument("--no-graph", action="store_true",
                    help="--decoder: time eager steps instead of HIP-graph replays")
    ap.add_argument("--model", action="store_true",
                    help="the C++ drop-in PhiTinyMoEModel::generate on the reference's model "
                         "shape (32 layers; writes a ~15 GiB model.bin to a temporary directory)")
    ap.add_argument("--no-extra", action="store_true",
                    help="config 3: skip timing the other layer shapes after the headline")
    ap.add_argument("--dropin", action="store_true",
                    help="the C++ drop-in PhiMoE::forward at the reference's layer shape, host "
                         "tensors in and out (PCIe-inclusive)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported "
              "(this build targets a single MI355X: one GPU's share of the expert "
              "GEMMs is what it times)",
              file=sys.stderr)
        sys.exit(2)
    if args.sgemm:
        sgemm_sweep(args)
        return
    if args.decoder:
        decoder_bench(args, load_pkg())
        return
    if args.dropin:
        dropin_bench(args)
        return
    if args.model:
        model_bench(args)
        return

    import numpy as np
    import torch

    cfg = CONFIGS[args.config]
    T, d, E, k, d_ff = cfg["T"], cfg["d"], cfg["E"], cfg["k"], cfg["d_ff"]
    if args.tokens is not None:
        T = args.tokens  # a batch-size point of the configuration's layer shape
    pkg = load_pkg()
    dev = torch.device("cuda:0")
    rms = cfg["norm"] == "rms"
    x, weights, y, idx, w, desc = build_layer(pkg, cfg, T, args.block, dev)
    ctx = pkg.Context(0)
    ctx.reserve(desc)
    spin_steps, elapsed, instrumented, kt = time_layer(ctx, desc, weights, x, y, idx, w,
                                                       args.warmup, args.steps)

    ms_per_step = 1e3 * elapsed / args.steps
    tokens_per_s = T * args.steps / elapsed
    counts = np.bincount(idx.cpu().numpy().ravel(), minlength=E)
    pairs = T * k
    flops_w13 = 2.0 * pairs * d * d_ff * 2
    flops_w2 = 2.0 * pairs * d_ff * d
    avg = {name: ms / n for name, (ms, n) in kt.items()}
    hbm = hbm_kernel_rates(avg, T, d, E, k, args.block, ctx.w2_splits(desc))
    w13_ms = avg["expert_w13_swiglu"]
    w2_ms = avg["expert_w2"]
    w13_tflops = flops_w13 / (w13_ms * 1e-3) / 1e12
    expert_tflops = (flops_w13 + flops_w2) / ((w13_ms + w2_ms) * 1e-3) / 1e12

    traffic = None
    tpath = os.path.join(ROOT, "profiles", f"traffic_{args.config}.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("expert_w13_swiglu_bytes_per_launch")

    cpu = None
    parity = None
    if args.cpu_seconds > 0:
        host = {n: (None if v is None else v.cpu().numpy()) for n, v in weights.items()}
        cpu, parity = cpu_baseline(x.cpu().numpy(), host, cfg,
                                   (y.cpu().numpy(), idx.cpu().numpy()), args.cpu_seconds)

    out = {
        "metric": METRIC,
        "value": tokens_per_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded torch.randn: x ~ N(0,1), weights ~ N(0,0.02))",
        "config": {"workload": cfg["workload"], "tokens": T, "d_model": d, "experts": E,
                   "top_k": k, "d_ff": d_ff,
                   "router": ("quantised top-2, weights 1/2 (PhiMoE::route)"
                              if cfg.get("router") == "phi_quant"
                              else "softmax over selected top-k"),
                   "expert": "SwiGLU", "router_bias": (f"zipf(s={cfg['zipf']})"
                                                       if cfg["zipf"] else None),
                   "block": (f"y = x + MoE({'rms_norm' if rms else 'layer_norm'}(x))"
                             if args.block else None)},
        "expert_gemm_tflops": expert_tflops,
        "expert_gemm_frac_fp32_mfma_peak": expert_tflops / FP32_MFMA_PEAK_TFLOPS,
        "roofline": {
            "kernel": "expert_w13_swiglu",
            "bound": "mfma",
            "achieved": w13_tflops,
            "peak": FP32_MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": w13_tflops / FP32_MFMA_PEAK_TFLOPS,
            "traffic": traffic,
            "flops_per_launch": flops_w13,
        },
        "kernel_avg_ms": {n: round(v, 5) for n, v in sorted(avg.items())},
        "hbm_kernels": hbm,
        "expert_rows": counts.tolist(),
        "cpu_baseline": cpu,
        "cpu_sample_parity": parity,
        "spinup": f"{spin_steps} untimed forwards over {SPINUP_S:.1f} s before the warm-up steps",
        "timing": (f"ms_per_step from {args.steps} steps without per-kernel events; "
                   f"kernel_avg_ms and the roofline from HIP events over {args.steps} more "
                   f"steps ({1e3 * instrumented / args.steps:.3f} ms per instrumented step)"),
    }
    if args.config == "ref":
        # the reference's own per-layer expert GEMM times at this shape (RTX 3090)
        out["reference_gpu_gemm_ms"] = {n: round(v, 3) for n, v in REF_GEMM_MS.items()}
        out["speedup_vs_reference_gpu_gemms"] = {
            n: round(REF_GEMM_MS[n] / avg[n], 2) for n in REF_GEMM_MS if n in avg}
    ctx.close()
    if args.config == "c3" and args.tokens is None and not args.block and not args.no_extra:
        # the other layer shapes of the configurations, timed the same way in
        # this run (no CPU leg): the short-K expert GEMMs of config 5 and of the
        # reference's own layer, and config 4's skewed 64 experts
        del x, weights, y, idx, w
        torch.cuda.empty_cache()
        out["other_layer_shapes"] = {c: layer_point(pkg, c, dev, args.warmup, min(args.steps, 10))
                                     for c in ("c5", "ref", "c4")}
    print(json.dumps(out))


def build_layer(pkg, cfg, T, block, dev):
    """Seeded inputs, weights, outputs and the descriptor of one layer shape."""
    import torch
    d, E, k, d_ff = cfg["d"], cfg["E"], cfg["k"], cfg["d_ff"]
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn((T, d), device=dev, generator=g)
    weights = {
        "gate_w": torch.randn((E, d), device=dev, generator=g) * 0.02,
        "w1": torch.randn((E, d_ff, d), device=dev, generator=g) * 0.02,
        "w3": torch.randn((E, d_ff, d), device=dev, generator=g) * 0.02,
        "w2": torch.randn((E, d, d_ff), device=dev, generator=g) * 0.02,
        "expert_bias": None,
    }
    if cfg["zipf"] is not None:
        weights["expert_bias"] = torch.from_numpy(zipf_bias(E, cfg["zipf"])).to(dev)
    rms = cfg["norm"] == "rms"
    if block:
        weights["norm_w"] = 1 + 0.1 * torch.randn(d, device=dev, generator=g)
        weights["norm_b"] = None if rms else 0.1 * torch.randn(d, device=dev, generator=g)
    y = torch.empty((T, d), device=dev)
    idx = torch.empty((T, k), dtype=torch.int32, device=dev)
    w = torch.empty((T, k), device=dev)
    desc = pkg.make_desc(T, d, E, k, d_ff, act=pkg.ACT_SWIGLU,
                         router=(pkg.ROUTER_PHI_QUANT if cfg.get("router") == "phi_quant"
                                 else pkg.ROUTER_SOFTMAX_TOPK), contract=pkg.CONTRACT_FMA,
                         norm=(pkg.NORM_RMS if rms else pkg.NORM_LAYER) if block
                         else pkg.NORM_NONE,
                         norm_eps=NORM_EPS, residual=block)
    return x, weights, y, idx, w, desc


def time_layer(ctx, desc, weights, x, y, idx, w, warmup, steps):
    """Spin-up, warm-up, `steps` timed forwards without per-kernel events,
    then as many with HIP events around every launch (on the stream the
    kernels run on).  Returns (spin-up forwards, timed seconds, instrumented
    seconds, per-kernel times)."""
    import torch
    # spin-up: the GPU takes about a second of load to reach its full clock
    # (durations of short layers fall 10-20 % over the first second), so
    # forwards run for at least SPINUP_S before the warm-up steps
    spin_steps, t_spin = 0, time.perf_counter()
    while time.perf_counter() - t_spin < SPINUP_S:
        ctx.layer_forward(desc, weights, x, y, idx, w)
        torch.cuda.synchronize()
        spin_steps += 1
    for _ in range(warmup):
        ctx.layer_forward(desc, weights, x, y, idx, w)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        ctx.layer_forward(desc, weights, x, y, idx, w)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ctx.reset_timing()
    ctx.set_timing(True)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(steps):
        ctx.layer_forward(desc, weights, x, y, idx, w)
    torch.cuda.synchronize()
    instrumented = time.perf_counter() - t1
    ctx.set_timing(False)
    return spin_steps, elapsed, instrumented, ctx.kernel_times()


def layer_point(pkg, name, dev, warmup, steps):
    """One configuration's layer timed as the headline one is: tokens/s, the
    expert GEMMs' fraction of the fp32 MFMA peak, the w1/w3 roofline."""
    import torch
    cfg = CONFIGS[name]
    T, d, k, d_ff = cfg["T"], cfg["d"], cfg["k"], cfg["d_ff"]
    x, weights, y, idx, w, desc = build_layer(pkg, cfg, T, False, dev)
    ctx = pkg.Context(0)
    ctx.reserve(desc)
    _, elapsed, _, kt = time_layer(ctx, desc, weights, x, y, idx, w, warmup, steps)
    ctx.close()
    avg = {n: ms / c for n, (ms, c) in kt.items()}
    pairs = T * k
    f13, f2 = 2.0 * pairs * d * d_ff * 2, 2.0 * pairs * d_ff * d
    w13, w2 = avg["expert_w13_swiglu"], avg["expert_w2"]
    del x, weights, y, idx, w
    torch.cuda.empty_cache()
    return {"workload": cfg["workload"], "tokens": T, "ms_per_step": round(1e3 * elapsed / steps, 4),
            "tokens_per_s": round(T * steps / elapsed),
            "expert_gemm_frac_fp32_mfma_peak":
                round((f13 + f2) / ((w13 + w2) * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS, 4),
            "w13_frac_fp32_mfma_peak": round(f13 / (w13 * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS, 4),
            "kernel_avg_ms": {"expert_w13_swiglu": round(w13, 4), "expert_w2": round(w2, 4)},
            "steps": steps}


if __name__ == "__main__":
    main()
