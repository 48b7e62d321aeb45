// synth.cpp -- deterministic synthetic tensors (host only).  See cpb_synth.h.
#include "cpb_synth.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace {

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
inline uint64_t stream_key(uint64_t seed, uint64_t stream) {
    return mix64(mix64(seed + 0x632BE59BD9B4E019ull) ^ (stream * 0x9E3779B97F4A7C15ull + 0xD1B54A32D192ED03ull));
}
inline uint64_t word(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * 0x9E3779B97F4A7C15ull); }

// uniform in (0, 1): 53 random bits, offset by half an ulp so log() is finite
inline double unit(uint64_t w) { return ((double)(w >> 11) + 0.5) * (1.0 / 9007199254740992.0); }

template <class F>
void parallel_for(size_t n, size_t grain, F f) {
    unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if (n < grain * 2 || nt == 1) { f(0, n); return; }
    size_t chunks = std::min<size_t>(nt, (n + grain - 1) / grain);
    size_t per = (n + chunks - 1) / chunks;
    std::vector<std::thread> th;
    for (size_t c = 0; c < chunks; c++) {
        size_t a = c * per, b = std::min(n, a + per);
        if (a >= b) break;
        th.emplace_back([=] { f(a, b); });
    }
    for (auto& t : th) t.join();
}

inline float normal_at(uint64_t key, uint64_t i) {
    double u1 = unit(word(key, 2 * i)), u2 = unit(word(key, 2 * i + 1));
    return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
}

}  // namespace

extern "C" {

uint64_t cpb_synth_u64(uint64_t seed, uint64_t stream, uint64_t i) { return word(stream_key(seed, stream), i); }

uint16_t cpb_f32_to_half(float f) {
    uint32_t x; std::memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);           // rounds to inf
    if (ax < 0x38800000u) {                                              // half subnormal or zero
        if (ax < 0x33000000u) return (uint16_t)sign;                     // < 2^-25: rounds to 0
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        int shift = 126 - (int)(ax >> 23);                               // 14..24
        uint32_t r = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((ax >> 13) - (112u << 10));
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

void cpb_synth_mxfp4(uint8_t* out, size_t nblocks, int e_lo, int e_span, uint64_t seed, uint64_t stream) {
    uint64_t key = stream_key(seed, stream);
    if (e_span < 1) e_span = 1;
    parallel_for(nblocks, 1 << 16, [&](size_t a, size_t b) {
        for (size_t q = a; q < b; q++) {
            uint8_t* p = out + q * 17;
            uint64_t w0 = word(key, 3 * q), w1 = word(key, 3 * q + 1), w2 = word(key, 3 * q + 2);
            p[0] = (uint8_t)(e_lo + (int)(w2 % (uint64_t)e_span));
            std::memcpy(p + 1, &w0, 8);
            std::memcpy(p + 9, &w1, 8);
        }
    });
}

void cpb_synth_normal(float* out, size_t n, float mean, float sigma, uint64_t seed, uint64_t stream) {
    uint64_t key = stream_key(seed, stream);
    parallel_for(n, 1 << 15, [&](size_t a, size_t b) {
        for (size_t i = a; i < b; i++) out[i] = mean + sigma * normal_at(key, i);
    });
}

void cpb_synth_q4k(uint8_t* out, size_t nsuper, float dsig, uint64_t seed, uint64_t stream) {
    uint64_t key = stream_key(seed, stream);
    parallel_for(nsuper, 1 << 12, [&](size_t a, size_t b) {
        for (size_t s = a; s < b; s++) {
            uint8_t* p = out + s * 144;
            uint64_t base = s * 20;
            uint16_t d = cpb_f32_to_half(std::fabs(dsig * normal_at(key ^ 0x5151ull, 2 * s)));
            uint16_t dm = cpb_f32_to_half(std::fabs(dsig * normal_at(key ^ 0x5151ull, 2 * s + 1)));
            p[0] = (uint8_t)d; p[1] = (uint8_t)(d >> 8); p[2] = (uint8_t)dm; p[3] = (uint8_t)(dm >> 8);
            uint8_t buf[144];
            for (int k = 0; k < 18; k++) { uint64_t w = word(key, base + k); std::memcpy(buf + 8 * k, &w, 8); }
            std::memcpy(p + 4, buf, 140);
        }
    });
}

void cpb_synth_q6k(uint8_t* out, size_t nsuper, float dsig, uint64_t seed, uint64_t stream) {
    uint64_t key = stream_key(seed, stream);
    parallel_for(nsuper, 1 << 12, [&](size_t a, size_t b) {
        for (size_t s = a; s < b; s++) {
            uint8_t* p = out + s * 210;
            uint64_t base = s * 27;
            uint8_t buf[216];
            for (int k = 0; k < 27; k++) { uint64_t w = word(key, base + k); std::memcpy(buf + 8 * k, &w, 8); }
            std::memcpy(p, buf, 208);
            uint16_t d = cpb_f32_to_half(std::fabs(dsig * normal_at(key ^ 0x6161ull, s)));
            p[208] = (uint8_t)d; p[209] = (uint8_t)(d >> 8);
        }
    });
}

void cpb_synth_zipf_bias(float* out, int ne, float s, uint64_t seed, uint64_t stream) {
    uint64_t key = stream_key(seed, stream);
    std::vector<int> perm(ne);
    for (int i = 0; i < ne; i++) perm[i] = i;
    for (int i = ne - 1; i > 0; i--) {                       // Fisher-Yates
        int j = (int)(word(key, (uint64_t)i) % (uint64_t)(i + 1));
        std::swap(perm[i], perm[j]);
    }
    double z = 0.0;
    for (int r = 1; r <= ne; r++) z += std::pow((double)r, -(double)s);
    for (int i = 0; i < ne; i++) {
        int r = perm[i] + 1;                                  // expert i gets rank r
        out[i] = (float)std::log(std::pow((double)r, -(double)s) / z);
    }
}

}  // extern "C"
