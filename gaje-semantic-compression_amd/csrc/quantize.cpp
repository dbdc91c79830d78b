// Writer-side quantisers (see quantize.h).
#include "quantize.h"

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstring>
#include <thread>

namespace gaje {

namespace {

template <class F>
void parallel_blocks(int64_t n, F f) {
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0) nt = 4;
    if (nt > 16) nt = 16;
    if (n < 4096) nt = 1;
    std::vector<std::thread> th;
    const int64_t per = (n + nt - 1) / nt;
    for (unsigned t = 0; t < nt; ++t) {
        const int64_t a = t * per, b = std::min<int64_t>(n, a + per);
        if (a >= b) break;
        th.emplace_back([=] { f(a, b); });
    }
    for (auto &x : th) x.join();
}

// f32::round (half away from zero) then clamp(lo, hi), then `as` an integer:
// NaN stays NaN through clamp and casts to 0.
inline float round_clamp(float v, float lo, float hi) {
    if (v != v) return 0.0f;
    const float r = std::round(v);
    return r < lo ? lo : r > hi ? hi : r;
}

}  // namespace

uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, exp = (x >> 23) & 0xFFu, mant = x & 0x7FFFFFu;
    if (exp == 0xFF) return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u | (mant >> 13) : 0));
    const int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        const uint32_t full = mant | 0x800000u;
        const int shift = 14 - e;
        uint32_t h = full >> shift;
        const uint32_t rem = full & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1u))) ++h;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)e << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;  // a carry into the exponent is the correct rounding
    return (uint16_t)(sign | h);
}

// Per block of 32: min and max by '<' and '>' from f32::MAX / f32::MIN,
// scale = (max - min) / 15, inv = 1 / scale when scale > 1e-7 (else every code
// is 0), q = round((w - min) * inv) clamped to 0..15, qs[k] = q(2k) | q(2k+1) << 4,
// then scale and min as f16.
void quantize_q4_0(const float *w, int64_t n, uint8_t *blocks) {
    parallel_blocks(n / 32, [&](int64_t a, int64_t b) {
        for (int64_t j = a; j < b; ++j) {
            const float *blk = w + j * 32;
            float mn = FLT_MAX, mx = -FLT_MAX;
            for (int k = 0; k < 32; ++k) {
                if (blk[k] < mn) mn = blk[k];
                if (blk[k] > mx) mx = blk[k];
            }
            const float scale = (mx - mn) / 15.0f;
            const bool live = scale > 1e-7f;
            const float inv = live ? 1.0f / scale : 0.0f;
            uint8_t *o = blocks + j * 20;
            for (int k = 0; k < 16; ++k) {
                const uint8_t q0 = live ? (uint8_t)round_clamp((blk[2 * k] - mn) * inv, 0.0f, 15.0f) : 0;
                const uint8_t q1 = live ? (uint8_t)round_clamp((blk[2 * k + 1] - mn) * inv, 0.0f, 15.0f) : 0;
                o[4 + k] = (uint8_t)(q0 | (q1 << 4));
            }
            const uint16_t hs = f32_to_f16(scale), hm = f32_to_f16(mn);
            memcpy(o, &hs, 2);
            memcpy(o + 2, &hm, 2);
        }
    });
}

// Per block of 32: scale = max|w| / 127 (from 0, by '>'), inv = 1 / scale when
// scale > 1e-7 (else every code is 0), q = round(w * inv) clamped to
// [-128, 127]; the scale stored as f16.
void quantize_q8_0(const float *w, int64_t n, uint8_t *blocks) {
    parallel_blocks(n / 32, [&](int64_t a, int64_t b) {
        for (int64_t j = a; j < b; ++j) {
            const float *blk = w + j * 32;
            float max_abs = 0.0f;
            for (int k = 0; k < 32; ++k) max_abs = std::fabs(blk[k]) > max_abs ? std::fabs(blk[k]) : max_abs;
            const float scale = max_abs / 127.0f;
            const bool live = scale > 1e-7f;
            const float inv = live ? 1.0f / scale : 0.0f;
            uint8_t *o = blocks + j * 34;
            for (int k = 0; k < 32; ++k) o[2 + k] = live ? (uint8_t)(int8_t)round_clamp(blk[k] * inv, -128.0f, 127.0f) : 0;
            const uint16_t hs = f32_to_f16(scale);
            memcpy(o, &hs, 2);
        }
    });
}

bool genomize_4bit(const float *w, int64_t n, int64_t block_size, float anchor_threshold, std::vector<uint8_t> &codes,
                   std::vector<float> &centroids, std::vector<uint8_t> &anchors) {
    const int64_t nb = block_size > 0 ? n / block_size : 0;
    // a density in (0, 1): the threshold is the (n * density)-th largest |w|
    float thr = anchor_threshold;
    if (anchor_threshold > 0.0f && anchor_threshold < 1.0f) {
        std::vector<float> a((size_t)n);
        for (int64_t i = 0; i < n; ++i) {
            if (w[i] != w[i]) return false;
            a[(size_t)i] = std::fabs(w[i]);
        }
        const int64_t top = (int64_t)((float)n * anchor_threshold);
        if (top < n) {
            std::nth_element(a.begin(), a.begin() + top, a.end(), [](float x, float y) { return x > y; });
            thr = a[(size_t)top];
        } else {
            thr = 0.0f;
        }
    }
    codes.assign((size_t)(nb * (block_size / 2)), 0);
    centroids.assign((size_t)(nb * 16), 0.0f);
    std::vector<uint32_t> idx;
    std::vector<uint16_t> val;
    for (int64_t b = 0; b < nb; ++b) {
        const float *blk = w + b * block_size;
        float mn = FLT_MAX, mx = -FLT_MAX;
        for (int64_t k = 0; k < block_size; ++k) {
            if (blk[k] < mn) mn = blk[k];
            if (blk[k] > mx) mx = blk[k];
        }
        const float step = (mx - mn) / 15.0f;
        float c[16];
        for (int j = 0; j < 16; ++j) {
            const float t = (float)j * step;  // j as f32 * step, then + min, each rounded
            c[j] = mn + t;
            centroids[(size_t)(b * 16 + j)] = c[j];
        }
        for (int64_t k = 0; k < block_size / 2; ++k) {
            uint8_t byte = 0;
            for (int s = 0; s < 2; ++s) {
                const int64_t e = 2 * k + s;
                const float v = blk[e];
                int best = 0;
                float best_d = FLT_MAX;
                for (int j = 0; j < 16; ++j) {
                    const float d = std::fabs(v - c[j]);
                    if (d < best_d) {  // strict: ties go to the lower centroid
                        best_d = d;
                        best = j;
                    }
                }
                byte |= (uint8_t)(s == 0 ? best << 4 : best);  // high nibble = even element
                if (anchor_threshold >= 0.0f && std::fabs(v) >= thr) {
                    idx.push_back((uint32_t)(b * block_size + e));
                    val.push_back(f32_to_f16(v));
                }
            }
            codes[(size_t)(b * (block_size / 2) + k)] = byte;
        }
    }
    // "GAJE", count, the u32 indices, the f16 values, then the two row pointers
    // {0, count} the reference writes (genomize.rs:373-376)
    const uint32_t cnt = (uint32_t)idx.size();
    anchors.assign(8 + (size_t)cnt * 6 + 16, 0);
    memcpy(anchors.data(), "GAJE", 4);
    memcpy(anchors.data() + 4, &cnt, 4);
    if (cnt) {
        memcpy(anchors.data() + 8, idx.data(), (size_t)cnt * 4);
        memcpy(anchors.data() + 8 + (size_t)cnt * 4, val.data(), (size_t)cnt * 2);
    }
    const uint64_t ptrs[2] = {0, cnt};
    memcpy(anchors.data() + 8 + (size_t)cnt * 6, ptrs, 16);
    return true;
}

}  // namespace gaje
