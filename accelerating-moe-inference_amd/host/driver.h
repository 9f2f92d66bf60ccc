// The driver's file formats and validation rules (src/main.cpp:144-520 of
// the reference), as functions a driver built on the drop-in calls: the
// variable-length inputs.bin, outputs.bin / decode outputs, the answer files
// and the -v rules.  Same formats, checks, messages and exception types
// (std::runtime_error for I/O and format errors).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "tensor.h"

namespace moe_driver {

// uint32 batch, uint32 max_seq_len, then per sequence uint32 len and int32
// ids[len]; 0 < len <= max_seq_len <= MAX_POSITION_EMBEDDINGS.
std::vector<std::vector<int>> read_inputs(const std::string& path, std::size_t& max_seq_len);
// uint32 batch, uint32 vocab, float logits[batch][vocab].
void write_outputs(const std::string& path, const Tensor& logits);
// uint32 batch, uint32 max_decode_tokens, uint32 vocab, uint32 lengths[batch],
// int32 ids[batch][max_decode_tokens] (-1 after a sequence's length),
// float logits[batch][max_decode_tokens][vocab].
void write_decode_outputs(const std::string& path, const Tensor& logits,
                          const std::vector<std::vector<int>>& generated_ids);
// The first batch * vocab floats of an answer file.
Tensor read_answers(const std::string& path, std::size_t batch, std::size_t vocab);

struct DecodeAnswers {
    std::vector<std::uint32_t> lengths;
    std::vector<std::int32_t> generated_ids;
    Tensor logits;
};
// The first `batch` sequences of a decode answer file (its header must have
// max_steps and vocab, and at least batch sequences).
DecodeAnswers read_decode_answers(const std::string& path, std::size_t batch,
                                  std::size_t max_steps, std::size_t vocab);

// -v: an element fails when it is NaN, or when both its absolute and its
// relative error exceed 3e-3; prints the max/mean absolute error and PASSED
// or the first mismatch.
bool validate(const Tensor& output, const Tensor& answer);
// -v -d: lengths and tokens must match exactly; step 0's logits by the rule
// of validate(); every later step's logit vector by its normalised mean
// absolute error (<= 7.5e-2) and Huber mean (<= 7.5e-4, delta 1e-2); any
// non-finite logit fails.
bool validate_decode(const Tensor& output, const std::vector<std::vector<int>>& generated_ids,
                     const DecodeAnswers& answer);

}  // namespace moe_driver
