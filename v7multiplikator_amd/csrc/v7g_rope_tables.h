// v7g_rope_tables.h -- the host RoPE table builders (v7g_rope_tables.cpp,
// compiled for the x86-64 host only: they use x87 instructions).
#pragma once
#include <vector>

namespace v7g {
// Plain frequencies base^(-j/half), j < half (rope type 0), as doubles.
std::vector<double> plain_freqs(int half, float base);
// Llama 3 scaled frequencies (rope type 1).
std::vector<double> llama3_freqs(int half, float base, float factor, float low_freq_factor, float high_freq_factor,
                                 int orig_max_pos);
// cos/sin tables [n_pos, freq.size()] from the frequencies.
void fill_tables(std::vector<float> &c, std::vector<float> &s, int n_pos, const std::vector<double> &freq);
}  // namespace v7g
