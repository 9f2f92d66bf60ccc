#include "driver.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <fstream>
#include <stdexcept>

#include "config.h"

namespace moe_driver {
namespace {

template <class T>
bool get(std::istream& f, T& v) {
    return static_cast<bool>(f.read(reinterpret_cast<char*>(&v), sizeof(T)));
}

template <class T>
void put(std::ostream& f, const T& v) {
    f.write(reinterpret_cast<const char*>(&v), sizeof(T));
}

// |actual - expected| and the relative error the reference's rule uses
// (absolute where |expected| <= 1e-8).
template <class F>
void errors(F actual, F expected, F& abs_error, F& rel_error) {
    abs_error = std::fabs(actual - expected);
    rel_error = std::fabs(expected) > F(1.0e-8) ? abs_error / std::fabs(expected) : abs_error;
}

}  // namespace

// src/main.cpp:144-183
std::vector<std::vector<int>> read_inputs(const std::string& path, std::size_t& max_seq_len) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open input: " + path);
    std::uint32_t batch = 0, max_seq = 0;
    const bool ok = get(f, batch) && get(f, max_seq);
    if (!ok || batch == 0 || max_seq == 0 || max_seq > apss26::MAX_POSITION_EMBEDDINGS)
        throw std::runtime_error("invalid input header");
    max_seq_len = max_seq;
    std::vector<std::vector<int>> ids(batch);
    for (std::vector<int>& row : ids) {
        std::uint32_t len = 0;
        if (!get(f, len) || len == 0 || len > max_seq)
            throw std::runtime_error("invalid sequence length in input");
        row.resize(len);
        for (int& token : row) {
            std::int32_t value = 0;
            if (!get(f, value)) throw std::runtime_error("truncated input");
            token = value;
        }
    }
    return ids;
}

// src/main.cpp:185-195
void write_outputs(const std::string& path, const Tensor& logits) {
    std::ofstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open output: " + path);
    put(f, static_cast<std::uint32_t>(logits.size(0)));
    put(f, static_cast<std::uint32_t>(logits.size(1)));
    f.write(reinterpret_cast<const char*>(logits.data()),
            static_cast<std::streamsize>(logits.size() * sizeof(float)));
    if (!f) throw std::runtime_error("failed while writing output: " + path);
}

// src/main.cpp:197-241
void write_decode_outputs(const std::string& path, const Tensor& logits,
                          const std::vector<std::vector<int>>& generated_ids) {
    if (logits.ndim() != 3 || logits.size(0) != generated_ids.size())
        throw std::runtime_error("invalid decode output shape");
    std::ofstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open output: " + path);
    const std::size_t steps = logits.size(1);
    put(f, static_cast<std::uint32_t>(logits.size(0)));
    put(f, static_cast<std::uint32_t>(steps));
    put(f, static_cast<std::uint32_t>(logits.size(2)));
    for (const std::vector<int>& row : generated_ids) {
        if (row.size() > steps) throw std::runtime_error("generated sequence exceeds decode limit");
        put(f, static_cast<std::uint32_t>(row.size()));
    }
    for (const std::vector<int>& row : generated_ids)
        for (std::size_t s = 0; s < steps; ++s)
            put(f, static_cast<std::int32_t>(s < row.size() ? row[s] : -1));
    f.write(reinterpret_cast<const char*>(logits.data()),
            static_cast<std::streamsize>(logits.size() * sizeof(float)));
    if (!f) throw std::runtime_error("failed while writing output: " + path);
}

// src/main.cpp:243-264
Tensor read_answers(const std::string& path, std::size_t batch, std::size_t vocab) {
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f) throw std::runtime_error("cannot open answer: " + path);
    const auto want = static_cast<std::streamsize>(batch * vocab * sizeof(float));
    const std::streamsize have = f.tellg();
    if (have < want)
        throw std::runtime_error("invalid answer size: expected at least " + std::to_string(want) +
                                 " bytes, got " + std::to_string(static_cast<long long>(have)));
    f.seekg(0, std::ios::beg);
    Tensor answers({batch, vocab});
    f.read(reinterpret_cast<char*>(answers.data()), want);
    if (!f) throw std::runtime_error("failed while reading answer: " + path);
    return answers;
}

// src/main.cpp:272-321
DecodeAnswers read_decode_answers(const std::string& path, std::size_t batch,
                                  std::size_t max_steps, std::size_t vocab) {
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f) throw std::runtime_error("cannot open decode answer: " + path);
    const std::streamsize bytes = f.tellg();
    constexpr std::streamsize header = 3 * sizeof(std::uint32_t);
    if (bytes < header) throw std::runtime_error("decode answer is too small");
    f.seekg(0, std::ios::beg);
    std::uint32_t fb = 0, fs = 0, fv = 0;
    const bool ok = get(f, fb) && get(f, fs) && get(f, fv);
    if (!ok || fb < batch || fs != max_steps || fv != vocab)
        throw std::runtime_error("decode answer header mismatch");
    const std::streamoff lengths_at = header;
    const std::streamoff ids_at = lengths_at + std::streamoff(fb) * sizeof(std::uint32_t);
    const std::streamoff logits_at = ids_at + std::streamoff(fb) * fs * sizeof(std::int32_t);
    if (bytes < logits_at + std::streamoff(fb) * fs * fv * std::streamoff(sizeof(float)))
        throw std::runtime_error("decode answer is truncated");
    DecodeAnswers a;
    a.lengths.resize(batch);
    a.generated_ids.resize(batch * max_steps);
    a.logits = Tensor({batch, max_steps, vocab});
    f.seekg(lengths_at, std::ios::beg);
    f.read(reinterpret_cast<char*>(a.lengths.data()),
           static_cast<std::streamsize>(batch * sizeof(std::uint32_t)));
    f.seekg(ids_at, std::ios::beg);
    f.read(reinterpret_cast<char*>(a.generated_ids.data()),
           static_cast<std::streamsize>(batch * max_steps * sizeof(std::int32_t)));
    f.seekg(logits_at, std::ios::beg);
    f.read(reinterpret_cast<char*>(a.logits.data()),
           static_cast<std::streamsize>(batch * max_steps * vocab * sizeof(float)));
    if (!f) throw std::runtime_error("failed while reading decode answer");
    return a;
}

// src/main.cpp:323-363
bool validate(const Tensor& output, const Tensor& answer) {
    if (output.shape() != answer.shape()) throw std::runtime_error("output/answer shape mismatch");
    constexpr float threshold = 3.0e-3f;
    float max_abs = 0.0f, mean_abs = 0.0f;
    std::size_t first_bad = output.size();
    for (std::size_t i = 0; i < output.size(); ++i) {
        float abs_error = 0.0f, rel_error = 0.0f;
        errors(output[i], answer[i], abs_error, rel_error);
        max_abs = std::max(max_abs, abs_error);
        mean_abs += abs_error;
        if (first_bad == output.size() &&
            (std::isnan(output[i]) || (abs_error > threshold && rel_error > threshold)))
            first_bad = i;
    }
    mean_abs /= static_cast<float>(output.size());
    std::fprintf(stdout, "Validation max abs diff: %g\n", max_abs);
    std::fprintf(stdout, "Validation mean abs diff: %g\n", mean_abs);
    if (first_bad == output.size()) {
        std::fprintf(stdout, "Validation: PASSED!\n");
        return true;
    }
    const std::size_t vocab = output.size(1);
    std::fprintf(stdout, "Validation: FAILED! First mismatch at [%zu, %zu] (output=%g, answer=%g)\n",
                 first_bad / vocab, first_bad % vocab, output[first_bad], answer[first_bad]);
    return false;
}

// src/main.cpp:365-520 (the build without USE_TC)
bool validate_decode(const Tensor& output, const std::vector<std::vector<int>>& generated_ids,
                     const DecodeAnswers& answer) {
    if (output.shape() != answer.logits.shape() || generated_ids.size() != answer.lengths.size())
        throw std::runtime_error("decode output/answer shape mismatch");
    constexpr double step0_threshold = 3.0e-3, mae_threshold = 7.5e-2, huber_delta = 1.0e-2,
                     huber_threshold = 7.5e-4;
    double max_abs = 0.0, mean_abs = 0.0;
    std::size_t compared = 0;
    const std::size_t steps = answer.logits.size(1), vocab = output.size(2);
    auto summary = [&] {
        std::fprintf(stdout, "Validation max abs diff: %g\nValidation mean abs diff: %g\n", max_abs,
                     compared == 0 ? 0.0 : mean_abs / static_cast<double>(compared));
    };
    for (std::size_t b = 0; b < generated_ids.size(); ++b) {
        if (generated_ids[b].size() != answer.lengths[b]) {
            std::fprintf(stdout,
                         "Validation: FAILED! Generated length mismatch at sequence %zu "
                         "(output=%zu, answer=%u)\n",
                         b, generated_ids[b].size(), answer.lengths[b]);
            return false;
        }
        for (std::size_t s = 0; s < generated_ids[b].size(); ++s) {
            const std::int32_t want = answer.generated_ids[b * steps + s];
            if (generated_ids[b][s] != want) {
                std::fprintf(stdout,
                             "Validation: FAILED! Token mismatch at [%zu, %zu] (output=%d, "
                             "answer=%d)\n",
                             b, s, generated_ids[b][s], want);
                return false;
            }
            double norm_sum = 0.0, huber_sum = 0.0;
            for (std::size_t v = 0; v < vocab; ++v) {
                const double actual = output.at(b, s, v), expected = answer.logits.at(b, s, v);
                if (!std::isfinite(actual) || !std::isfinite(expected)) {
                    std::fprintf(stdout,
                                 "Validation: FAILED! Non-finite decode logit at [%zu, %zu, %zu]\n",
                                 b, s, v);
                    return false;
                }
                double abs_error = 0.0, rel_error = 0.0;
                errors(actual, expected, abs_error, rel_error);
                max_abs = std::max(max_abs, abs_error);
                mean_abs += abs_error;
                ++compared;
                if (s == 0 && abs_error > step0_threshold && rel_error > step0_threshold) {
                    summary();
                    std::fprintf(stdout,
                                 "Validation: FAILED! Prefill-logit mismatch at [%zu, %zu, %zu] "
                                 "(output=%g, answer=%g)\n",
                                 b, s, v, actual, expected);
                    return false;
                }
                if (s > 0) {
                    const double n = abs_error / (1.0 + std::fabs(expected));
                    norm_sum += n;
                    huber_sum += n <= huber_delta ? 0.5 * n * n : huber_delta * (n - 0.5 * huber_delta);
                }
            }
            if (s > 0) {
                const double mae = norm_sum / static_cast<double>(vocab);
                const double huber = huber_sum / static_cast<double>(vocab);
                if (mae > mae_threshold || huber > huber_threshold) {
                    summary();
                    std::fprintf(stdout,
                                 "Validation: FAILED! Decode vector mismatch at [%zu, %zu] "
                                 "(normalized MAE=%g, Huber=%g)\n",
                                 b, s, mae, huber);
                    return false;
                }
            }
        }
    }
    summary();
    std::fprintf(stdout, "Validation: PASSED!\n");
    return true;
}

}  // namespace moe_driver
