// Test shim: drives the C++ drop-in API (Tensor, tensor_ops, ModelLoader,
// Linear, PhiMLP, PhiMoE) exactly as reference code would, and exposes each
// scenario as an extern "C" function for tests/test_dropin.py (ctypes).
// Exceptions come back as codes: 1 invalid_argument, 2 runtime_error,
// 3 logic_error, 4 out_of_range, 5 other; shim_error() holds the message.
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "driver.h"
#include "layer.h"
#include "model.h"
#include "model_loader.h"
#include "tensor.h"

namespace {

thread_local std::string g_err;

template <class F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::invalid_argument& e) {
        g_err = e.what();
        return 1;
    } catch (const std::out_of_range& e) {
        g_err = e.what();
        return 4;
    } catch (const std::logic_error& e) {
        g_err = e.what();
        return 3;
    } catch (const std::runtime_error& e) {
        g_err = e.what();
        return 2;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 5;
    }
}

void expect(bool ok, const char* what) {
    if (!ok) throw std::runtime_error(std::string("expectation failed: ") + what);
}

template <class E, class F>
void expect_throw(F&& f, const char* what) {
    try {
        f();
    } catch (const E&) {
        return;
    }
    throw std::runtime_error(std::string("expected exception: ") + what);
}

Tensor make(const float* p, std::vector<std::size_t> shape) {
    Tensor t(std::move(shape));
    std::memcpy(t.data(), p, t.size() * sizeof(float));
    return t;
}

}  // namespace

extern "C" {

const char* shim_error() { return g_err.c_str(); }

// Tensor semantics of the reference's tensor.h:7-58.  Pinned allocation
// needs the HIP runtime to see a device, so it is checked only on request.
int shim_tensor_semantics(int with_pinned) {
    return guarded([&] {
        Tensor t({2, 3});
        expect(t.size() == 6 && t.ndim() == 2 && t.size(1) == 3, "shape");
        for (std::size_t i = 0; i < 6; ++i) expect(t[i] == 0.0f, "zero-initialised");
        expect_throw<std::out_of_range>([&] { (void)t.size(2); }, "size(dim) past rank");
        t.at(1, 2) = 5.0f;
        expect(t[5] == 5.0f, "row-major at()");
        expect_throw<std::out_of_range>([&] { (void)t.at(2, 0); }, "at() out of range");
        expect_throw<std::invalid_argument>([&] { (void)t.at(1); }, "at() rank mismatch");
        Tensor c = t;
        c.at(0, 0) = 1.0f;
        expect(t.at(0, 0) == 0.0f && c.at(1, 2) == 5.0f, "deep copy");
        Tensor m = std::move(c);
        expect(c.size() == 0 && c.data() == nullptr && m.at(0, 0) == 1.0f, "move");
        m.reshape({3, 2});
        expect(m.size(0) == 3 && m.at(2, 1) == 5.0f, "reshape");
        expect_throw<std::invalid_argument>([&] { m.reshape({4}); }, "reshape size change");
        m.reshape_within_capacity({1, 2});
        expect(m.size() == 2 && m.capacity() == 6, "reshape within capacity");
        expect_throw<std::invalid_argument>([&] { m.reshape_within_capacity({7}); },
                                            "reshape past capacity");
        m.fill(2.5f);
        expect(m[0] == 2.5f && m[1] == 2.5f, "fill");
        if (with_pinned) {
            Tensor p({4}, Tensor::Alloc::Pinned);
            p.at(3) = 1.0f;
            Tensor pc = p;
            expect(p.alloc() == Tensor::Alloc::Pinned && pc.alloc() == Tensor::Alloc::Host &&
                       pc.at(3) == 1.0f,
                   "copy of pinned is host");
        }
    });
}

int shim_loader_shape(const char* path, const char* name, int64_t* dims, int* ndim) {
    return guarded([&] {
        ModelLoader l(path);
        expect(l.has(name), "has()");
        const auto& s = l.shape(name);
        *ndim = static_cast<int>(s.size());
        for (std::size_t i = 0; i < s.size(); ++i) dims[i] = static_cast<int64_t>(s[i]);
    });
}

int shim_loader_load(const char* path, const char* name, float* out, int64_t n) {
    return guarded([&] {
        ModelLoader l(path);
        const Tensor t = l.load(name);
        expect(static_cast<int64_t>(t.size()) == n, "element count");
        std::memcpy(out, t.data(), t.size() * sizeof(float));
    });
}

int shim_matmul_transposed(const float* a, int64_t m, int64_t k, const float* b, int64_t n,
                           float* c) {
    return guarded([&] {
        Tensor A = make(a, {size_t(m), size_t(k)}), B = make(b, {size_t(n), size_t(k)});
        Tensor C({size_t(m), size_t(n)});
        tensor_ops::matmul_transposed(A, B, C);
        std::memcpy(c, C.data(), C.size() * sizeof(float));
    });
}

int shim_matmul(const float* a, int64_t m, int64_t k, const float* b, int64_t n, float* c) {
    return guarded([&] {
        Tensor A = make(a, {size_t(m), size_t(k)}), B = make(b, {size_t(k), size_t(n)});
        Tensor C({size_t(m), size_t(n)});
        tensor_ops::matmul(A, B, C);
        std::memcpy(c, C.data(), C.size() * sizeof(float));
    });
}

int shim_matmul_bad_shape() {
    return guarded([] {
        Tensor A({2, 3}), B({4, 5}), C({2, 4});
        tensor_ops::matmul_transposed(A, B, C);
    });
}

int shim_silu_mul(const float* x, const float* u, int64_t n, float* s, float* p) {
    return guarded([&] {
        Tensor X = make(x, {size_t(n)}), U = make(u, {size_t(n)}), S({size_t(n)}), P({size_t(n)});
        tensor_ops::silu(X, S);
        tensor_ops::mul(S, U, P);
        std::memcpy(s, S.data(), n * sizeof(float));
        std::memcpy(p, P.data(), n * sizeof(float));
    });
}

// Declared by the reference's header, defined nowhere: logic_error.
int shim_outside_op() {
    return guarded([] {
        Tensor x({2, 8}), y({2, 8});
        tensor_ops::softmax_last_dim(x, y);
    });
}

// Shape errors of the adds and RoPE, raised before any device work:
// 1 add, 2 bias rank, 3 bias width, 4 rope width, 5 rope odd head_dim,
// 6 rope seq_len past the rows (out_of_range).
int shim_elementwise_bad_shape(int which) {
    return guarded([&] {
        Tensor a({2, 4}), b({3, 4}), bias2({1, 4}), bias3({3});
        Tensor q({4, 16}), k({4, 8});
        switch (which) {
            case 1: tensor_ops::add_inplace(a, b); break;
            case 2: tensor_ops::add_bias_inplace(a, bias2); break;
            case 3: tensor_ops::add_bias_inplace(a, bias3); break;
            case 4: tensor_ops::apply_rope(q, k, 4, 2, 2, 8, 1e4f); break;
            case 5: tensor_ops::apply_rope(q, k, 4, 2, 1, 8 + 1, 1e4f); break;
            case 6: tensor_ops::apply_rope(q, k, 5, 2, 1, 8, 1e4f); break;
        }
    });
}

// a += b, then a += bias (rows x cols), through tensor_ops.
int shim_add_and_bias(const float* a, const float* b, const float* bias, int64_t rows,
                      int64_t cols, float* out) {
    return guarded([&] {
        Tensor A = make(a, {size_t(rows), size_t(cols)}), B = make(b, {size_t(rows), size_t(cols)}),
               Bias = make(bias, {size_t(cols)});
        tensor_ops::add_inplace(A, B);
        tensor_ops::add_bias_inplace(A, Bias);
        std::memcpy(out, A.data(), rows * cols * sizeof(float));
    });
}

// tensor_ops::apply_rope on q [rows, q_heads*hd], k [rows, kv_heads*hd].
int shim_rope(float* q, float* k, int64_t rows, int64_t seq_len, int64_t q_heads,
              int64_t kv_heads, int64_t hd, float theta) {
    return guarded([&] {
        Tensor Q = make(q, {size_t(rows), size_t(q_heads * hd)}),
               K = make(k, {size_t(rows), size_t(kv_heads * hd)});
        tensor_ops::apply_rope(Q, K, size_t(seq_len), size_t(q_heads), size_t(kv_heads),
                               size_t(hd), theta);
        std::memcpy(q, Q.data(), Q.size() * sizeof(float));
        std::memcpy(k, K.data(), K.size() * sizeof(float));
    });
}

int shim_layer_norm_bad_shape() {
    return guarded([] {
        Tensor x({2, 4}), w({3}), b({4}), y({2, 4});
        tensor_ops::layer_norm(x, w, b, 1e-5f, y);
    });
}

int shim_layer_norm(const float* x, int64_t rows, int64_t h, const float* w, const float* b,
                    float eps, float* y) {
    return guarded([&] {
        Tensor X = make(x, {size_t(rows), size_t(h)}), W = make(w, {size_t(h)}),
               B = make(b, {size_t(h)}), Y({size_t(rows), size_t(h)});
        tensor_ops::layer_norm(X, W, B, eps, Y);
        std::memcpy(y, Y.data(), rows * h * sizeof(float));
    });
}

int shim_linear(const char* path, const char* weight, const char* bias, const float* x,
                int64_t rows, int64_t in, float* y, int64_t out) {
    return guarded([&] {
        ModelLoader l(path);
        Linear lin(l, weight, bias);
        Tensor X = make(x, {size_t(rows), size_t(in)}), Y;
        lin.forward(X, Y);
        expect(Y.ndim() == 2 && Y.size(0) == size_t(rows) && Y.size(1) == size_t(out), "y shape");
        std::memcpy(y, Y.data(), Y.size() * sizeof(float));
    });
}

int shim_mlp(const char* path, const char* prefix, const float* x, int64_t rows, int64_t h,
             float* y) {
    return guarded([&] {
        ModelLoader l(path);
        PhiMLP mlp(l, prefix);
        Tensor X = make(x, {size_t(rows), size_t(h)}), Y;
        mlp.forward(X, Y);
        expect(Y.shape() == X.shape(), "y shaped like x");
        std::memcpy(y, Y.data(), Y.size() * sizeof(float));
    });
}

int shim_moe(const char* path, int64_t layer, int contract, const float* x, int64_t rows,
             int64_t h, float* y, int32_t* topk) {
    return guarded([&] {
        ModelLoader l(path);
        PhiMoE moe(l, size_t(layer), contract);
        Tensor X = make(x, {size_t(rows), size_t(h)}), Y;
        std::vector<int32_t> idx;
        moe.forward(X, Y, &idx);
        expect(Y.ndim() == 2 && Y.size(0) == size_t(rows) && Y.size(1) == size_t(h), "y shape");
        std::memcpy(y, Y.data(), Y.size() * sizeof(float));
        std::memcpy(topk, idx.data(), idx.size() * sizeof(int32_t));
    });
}

// Host-to-host time of PhiMoE::forward (the drop-in's PCIe copies included):
// builds the layer once, runs `warmup` untimed and `iters` timed forwards of
// x [rows, h], and returns the mean milliseconds per forward.
int shim_moe_time(const char* path, int64_t layer, const float* x, int64_t rows, int64_t h,
                  int64_t warmup, int64_t iters, double* ms) {
    return guarded([&] {
        if (iters <= 0 || warmup < 0)
            throw std::invalid_argument("iters must be > 0 and warmup >= 0");
        ModelLoader l(path);
        PhiMoE moe(l, size_t(layer));
        Tensor X = make(x, {size_t(rows), size_t(h)}), Y;
        for (int64_t i = 0; i < warmup; ++i) moe.forward(X, Y);
        const auto t0 = std::chrono::steady_clock::now();
        for (int64_t i = 0; i < iters; ++i) moe.forward(X, Y);
        const auto t1 = std::chrono::steady_clock::now();
        *ms = std::chrono::duration<double, std::milli>(t1 - t0).count() / double(iters);
    });
}

// PhiAttention / PhiDecoderLayer of layer `layer` on one sequence x [s, h].
int shim_attention(const char* path, int64_t layer, const float* x, int64_t s, int64_t h,
                   float* y) {
    return guarded([&] {
        ModelLoader l(path);
        PhiAttention att(l, size_t(layer));
        Tensor X = make(x, {size_t(s), size_t(h)}), Y;
        att.forward(X, Y);
        expect(Y.ndim() == 2 && Y.size(0) == size_t(s) && Y.size(1) == size_t(h), "y shape");
        std::memcpy(y, Y.data(), Y.size() * sizeof(float));
    });
}

int shim_decoder_layer(const char* path, int64_t layer, const float* x, int64_t s, int64_t h,
                       float* y) {
    return guarded([&] {
        ModelLoader l(path);
        PhiDecoderLayer dec(l, size_t(layer));
        Tensor X = make(x, {size_t(s), size_t(h)}), Y;
        dec.forward(X, Y);
        expect(Y.ndim() == 2 && Y.size(0) == size_t(s) && Y.size(1) == size_t(h), "y shape");
        std::memcpy(y, Y.data(), Y.size() * sizeof(float));
    });
}

// ---- PhiTinyMoEModel: sequences as lengths + concatenated ids.
namespace {
std::vector<std::vector<int>> unpack(const int32_t* lens, const int32_t* ids, int64_t batch) {
    std::vector<std::vector<int>> seqs(static_cast<std::size_t>(batch));
    std::size_t at = 0;
    for (int64_t b = 0; b < batch; ++b) {
        seqs[b].assign(ids + at, ids + at + lens[b]);
        at += static_cast<std::size_t>(lens[b]);
    }
    return seqs;
}
}  // namespace

int shim_model_generate(const char* path, const int32_t* lens, const int32_t* ids, int64_t batch,
                        float* logits, int64_t vocab) {
    return guarded([&] {
        PhiTinyMoEModel m(path);
        expect(m.vocab_size() == size_t(vocab), "vocab");
        Tensor L;
        m.generate(unpack(lens, ids, batch), L);
        expect(L.ndim() == 2 && L.size(0) == size_t(batch) && L.size(1) == size_t(vocab), "shape");
        std::memcpy(logits, L.data(), L.size() * sizeof(float));
        // again, on the model's warmed-up scratch: the same bits
        Tensor L2;
        m.generate(unpack(lens, ids, batch), L2);
        expect(std::memcmp(L.data(), L2.data(), L.size() * sizeof(float)) == 0, "repeat call");
        // forward() of one sequence is generate() of a batch of one
        Tensor one;
        m.forward(unpack(lens, ids, 1)[0], one);
        expect(one.ndim() == 2 && one.size(0) == 1, "forward shape");
        for (std::size_t v = 0; v < size_t(vocab); ++v)
            expect(std::fabs(one[v] - L[v]) <= 1e-4f * (1.0f + std::fabs(L[v])), "forward == row 0");
    });
}

// Times PhiTinyMoEModel: construction from the file (load_s, seconds) and
// generate() over the batch (ms per call, after `warmup` calls).  When
// `logits` is not null it receives the last call's [batch, vocab] logits.
int shim_model_time(const char* path, const int32_t* lens, const int32_t* ids, int64_t batch,
                    int64_t warmup, int64_t iters, double* load_s, double* ms, float* logits) {
    return guarded([&] {
        if (iters <= 0 || warmup < 0)
            throw std::invalid_argument("iters must be > 0 and warmup >= 0");
        const auto t0 = std::chrono::steady_clock::now();
        PhiTinyMoEModel m(path);
        const auto t1 = std::chrono::steady_clock::now();
        *load_s = std::chrono::duration<double>(t1 - t0).count();
        const std::vector<std::vector<int>> seqs = unpack(lens, ids, batch);
        Tensor L;
        for (int64_t i = 0; i < warmup; ++i) m.generate(seqs, L);
        const auto t2 = std::chrono::steady_clock::now();
        for (int64_t i = 0; i < iters; ++i) m.generate(seqs, L);
        const auto t3 = std::chrono::steady_clock::now();
        *ms = std::chrono::duration<double, std::milli>(t3 - t2).count() / double(iters);
        if (logits != nullptr) std::memcpy(logits, L.data(), L.size() * sizeof(float));
    });
}

int shim_model_decode(const char* path, const int32_t* lens, const int32_t* ids, int64_t batch,
                      int64_t max_new, float* logits, int32_t* gen_lens, int32_t* gen_ids) {
    return guarded([&] {
        PhiTinyMoEModel m(path);
        Tensor L;
        std::vector<std::vector<int>> gen;
        m.generate_decode(unpack(lens, ids, batch), size_t(max_new), L, gen);
        std::memcpy(logits, L.data(), L.size() * sizeof(float));
        for (int64_t b = 0; b < batch; ++b) {
            gen_lens[b] = static_cast<int32_t>(gen[b].size());
            for (int64_t s = 0; s < max_new; ++s)
                gen_ids[b * max_new + s] = s < int64_t(gen[b].size()) ? gen[b][s] : -1;
        }
    });
}

// Input errors of generate(): 1 empty batch, 2 empty sequence, 3 token past
// the vocabulary, 4 sequence longer than MAX_POSITION_EMBEDDINGS.
int shim_model_bad_input(const char* path, int which) {
    return guarded([&] {
        PhiTinyMoEModel m(path);
        Tensor L;
        std::vector<std::vector<int>> seqs;
        if (which == 2) seqs = {{1, 2}, {}};
        if (which == 3) seqs = {{1, int(m.vocab_size())}};
        if (which == 4) seqs = {std::vector<int>(apss26::MAX_POSITION_EMBEDDINGS + 1, 1)};
        m.generate(seqs, L);
    });
}

// ---- driver formats
int shim_read_inputs(const char* path, int64_t cap, int32_t* lens, int32_t* ids, int64_t* batch,
                     int64_t* max_seq) {
    return guarded([&] {
        std::size_t ms = 0;
        const auto seqs = moe_driver::read_inputs(path, ms);
        *batch = int64_t(seqs.size());
        *max_seq = int64_t(ms);
        std::size_t at = 0;
        for (std::size_t b = 0; b < seqs.size(); ++b) {
            lens[b] = int32_t(seqs[b].size());
            for (int t : seqs[b]) {
                expect(int64_t(at) < cap, "capacity");
                ids[at++] = t;
            }
        }
    });
}

int shim_write_outputs(const char* path, const float* logits, int64_t batch, int64_t vocab) {
    return guarded([&] {
        moe_driver::write_outputs(path, make(logits, {size_t(batch), size_t(vocab)}));
    });
}

// validate(output, read_answers(answer_path)); *passed = the verdict.
int shim_validate(const char* answer_path, const float* output, int64_t batch, int64_t vocab,
                  int* passed) {
    return guarded([&] {
        const Tensor ans = moe_driver::read_answers(answer_path, size_t(batch), size_t(vocab));
        *passed = moe_driver::validate(make(output, {size_t(batch), size_t(vocab)}), ans) ? 1 : 0;
    });
}

int shim_write_decode(const char* path, const float* logits, const int32_t* gen_lens,
                      const int32_t* gen_ids, int64_t batch, int64_t steps, int64_t vocab) {
    return guarded([&] {
        std::vector<std::vector<int>> gen(static_cast<std::size_t>(batch));
        for (int64_t b = 0; b < batch; ++b) gen[b].assign(gen_ids + b * steps, gen_ids + b * steps + gen_lens[b]);
        moe_driver::write_decode_outputs(path, make(logits, {size_t(batch), size_t(steps), size_t(vocab)}), gen);
    });
}

// validate_decode(output, ids, read_decode_answers(answer_path)).
int shim_validate_decode(const char* answer_path, const float* logits, const int32_t* gen_lens,
                         const int32_t* gen_ids, int64_t batch, int64_t steps, int64_t vocab,
                         int* passed) {
    return guarded([&] {
        const auto ans = moe_driver::read_decode_answers(answer_path, size_t(batch), size_t(steps),
                                                         size_t(vocab));
        std::vector<std::vector<int>> gen(static_cast<std::size_t>(batch));
        for (int64_t b = 0; b < batch; ++b) gen[b].assign(gen_ids + b * steps, gen_ids + b * steps + gen_lens[b]);
        *passed = moe_driver::validate_decode(
                      make(logits, {size_t(batch), size_t(steps), size_t(vocab)}), gen, ans)
                      ? 1
                      : 0;
    });
}

}  // extern "C"
