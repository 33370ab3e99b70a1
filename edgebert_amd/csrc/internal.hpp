// internal.hpp -- helpers shared by the host-side translation units (not exported).
#pragma once
#include <cstdint>
#include <memory>
#include <vector>

struct ebh_tokenizer;
struct ebh_model;

namespace ebh {
// Record this thread's error message (returned by ebh_last_error) and return code.
__attribute__((visibility("hidden"), format(printf, 2, 3))) int set_error(int code,
                                                                          const char* fmt, ...);

// Element encodings of checkpoint tensors (safetensors dtypes F32, F16, BF16).
enum TensorKind : int { TENSOR_F32 = 0, TENSOR_F16 = 1, TENSOR_BF16 = 2 };

// Hand one tensor to a model before ebh_finalize (api.cpp): checked against
// the config's names and shapes; f32 data without `keep` is copied, data with
// `keep` (the owner of the memory, e.g. a mapped file) is referenced in place
// until ebh_finalize uploads it in its own encoding.
int put_tensor(ebh_model* m, const char* name, const void* data, int kind, const int64_t* shape, int32_t ndim,
               std::shared_ptr<const void> keep);

// Host tokenizer (tokenizer.cpp): encodings of n texts and the batch's padded
// length; their [n, S] ids / mask with the tokenizer's padding.
int tokenize_batch(const ebh_tokenizer* t, const char* const* texts, const int64_t* lens, int n, int nthreads,
                   std::vector<std::vector<int32_t>>& seqs, int* S_out);
void write_padded(const ebh_tokenizer* t, const std::vector<std::vector<int32_t>>& seqs, int S, int32_t* ids,
                  int32_t* mask);
}  // namespace ebh
