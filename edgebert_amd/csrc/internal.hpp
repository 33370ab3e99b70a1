// internal.hpp -- helpers shared by the host-side translation units (not exported).
#pragma once
#include <cstdint>
#include <vector>

struct ebh_tokenizer;

namespace ebh {
// Record this thread's error message (returned by ebh_last_error) and return code.
__attribute__((visibility("hidden"), format(printf, 2, 3))) int set_error(int code,
                                                                          const char* fmt, ...);

// Host tokenizer (tokenizer.cpp): encodings of n texts and the batch's padded
// length; their [n, S] ids / mask with the tokenizer's padding.
int tokenize_batch(const ebh_tokenizer* t, const char* const* texts, const int64_t* lens, int n, int nthreads,
                   std::vector<std::vector<int32_t>>& seqs, int* S_out);
void write_padded(const ebh_tokenizer* t, const std::vector<std::vector<int32_t>>& seqs, int S, int32_t* ids,
                  int32_t* mask);
}  // namespace ebh
