// Writer-side quantisers of the .gaje.flat formats (host code), restating the
// reference's Rust functions bit for bit: f16 conversions round to nearest
// even (half::f16::from_f32), f32::round rounds half away from zero, and a
// NaN cast to an integer is 0 (Rust's saturating `as`).
#pragma once

#include <cstdint>
#include <vector>

namespace gaje {

// IEEE binary32 -> binary16, round to nearest even.
uint16_t f32_to_f16(float f);

// quantize_q4_0_native (compute/quantize/python.rs:151-232): n % 32 == 0
// weights -> n / 32 Q4_0Blocks of 20 bytes.
void quantize_q4_0(const float *w, int64_t n, uint8_t *blocks);

// quantize_q8_0_native (compute/quantize/python.rs:235-300): n % 32 == 0
// weights -> n / 32 Q8_0Blocks of 34 bytes.
void quantize_q8_0(const float *w, int64_t n, uint8_t *blocks);

// genomize_4bit_core (compute/quantize/genomize.rs:286-382): n / block_size
// blocks of 16 linear centroids, codes high nibble first (n / 2 bytes over the
// whole blocks), and the "GAJE" anchor buffer (always written; anchors only
// when anchor_threshold >= 0).  Fails (false) for a density threshold in
// (0, 1) over data holding a NaN, whose sort order the reference leaves open.
bool genomize_4bit(const float *w, int64_t n, int64_t block_size, float anchor_threshold, std::vector<uint8_t> &codes,
                   std::vector<float> &centroids, std::vector<uint8_t> &anchors);

}  // namespace gaje
