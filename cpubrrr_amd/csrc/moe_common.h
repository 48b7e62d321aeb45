// moe_common.h -- shared device helpers for the MoE kernels (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>

#define CPB_DEV __device__ __forceinline__
#define CPB_DEV_HOST_INLINE __host__ __device__ inline

namespace cpb {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 15 MXFP4 blocks per k-part: a lane streams 15 x 16 B of nibbles plus one
// 16 B unit holding the 15 e8m0 bytes, i.e. 16 dwordx4 loads per k-part.
constexpr int kBlkPerPart = 15;
constexpr int kUnits = 16;
// k-parts (two wavefronts each) per MXFP4 expert-GEMV workgroup: K <= 8 x 15 x 32 = 3840
constexpr int kMaxParts = 8;

// v_perm_b32: byte i of the result = byte sel_i of {hi:lo} (0-3 lo, 4-7 hi).
CPB_DEV uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) { return __builtin_amdgcn_perm(hi, lo, sel); }

// e4m3 encoding of a small integer v (0, or |v| with at most 4 significant
// bits and below 2^9: exact)
constexpr uint32_t e4m3_int(int v) {
    if (v == 0) return 0;
    uint32_t s = v < 0 ? 0x80u : 0u, a = (uint32_t)(v < 0 ? -v : v);
    int E = 0;
    while ((a >> (E + 1)) != 0) E++;
    uint32_t m = E >= 3 ? (a >> (E - 3)) & 7u : (a << (3 - E)) & 7u;
    return s | ((uint32_t)(E + 7) << 3) | m;
}
// table dword of entries 4c .. 4c+3 of f
template <typename F>
constexpr uint32_t table4(F f, int c) {
    return f(4 * c) | (f(4 * c + 1) << 8) | (f(4 * c + 2) << 16) | (f(4 * c + 3) << 24);
}
constexpr uint32_t img_h_entry(int i) { return e4m3_int(32 * (i < 8 ? i : i - 16)); }   // nibble i = h & 15
constexpr uint32_t img_l_entry(int i) { return e4m3_int(2 * i); }                        // nibble i = l
// 16-entry byte-wise table lookup: entry (nibble of each byte at bit `sh`)
template <int SH>
CPB_DEV uint32_t nib_lookup(uint32_t v, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
    const uint32_t i7 = (v >> SH) & 0x07070707u;
    const uint32_t lo = perm(t1, t0, i7), hi = perm(t3, t2, i7);
    return perm(hi, lo, ((v >> (SH + 1)) & 0x04040404u) | 0x03020100u);
}
// e4m3 of 32*h and of 2*l for the four int8 bytes x = 16*h + l of v
CPB_DEV uint32_t img_hi(uint32_t v) {
    return nib_lookup<4>(v, table4(img_h_entry, 0), table4(img_h_entry, 1), table4(img_h_entry, 2), table4(img_h_entry, 3));
}
CPB_DEV uint32_t img_lo(uint32_t v) {
    return nib_lookup<0>(v, table4(img_l_entry, 0), table4(img_l_entry, 1), table4(img_l_entry, 2), table4(img_l_entry, 3));
}
CPB_DEV int sdot4(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }

// 2^(e-128) * xsb exactly as the reference computes tbl[e] * xsb, with tbl
// from 2f32.powi(e-128) (tbl[0] = 0: the powi intermediate overflows).
CPB_DEV float e8m0_scale(uint32_t e, float xsb) { return e == 0 ? 0.0f : ldexpf(xsb, (int)e - 128); }


// Q8 round: (v / sc).round() in the reference's fp32 (quotient correctly
// rounded, then half away from zero), clamped to +-127.  The quotient from
// the hardware reciprocal, y = v * rcp(sc), lies within 2^-15 of the IEEE
// one for |v / sc| <= 128 (rcp within 1 ulp, the product rounded once: a
// relative error below 1.5 * 2^-23, plus half an ulp of the IEEE quotient).
// Unless y lies within 2^-13 of a half-integer, both round to the same
// integer (and round-to-nearest-even of y agrees with half-away-from-zero);
// only there (about one value in four thousand) the IEEE quotient decides.
CPB_DEV bool q8_near_half(float y) { return fabsf(__builtin_amdgcn_fractf(fabsf(y)) - 0.5f) < 0x1p-13f; }
CPB_DEV int8_t q8_clamp(float r) { return (int8_t)(int)fminf(fmaxf(r, -127.0f), 127.0f); }
CPB_DEV int8_t q8_round(float v, float sc) {
    const float y = v * __builtin_amdgcn_rcpf(sc);
    float r = __builtin_rintf(y);
    if (q8_near_half(y)) r = roundf(v / sc);
    return q8_clamp(r);
}
// q8_round of 16 values with one (rarely taken) branch for the exact path;
// the bytes packed little-endian into q[0..3].
CPB_DEV void q8_round16(const float* v, float sc, uint32_t* q) {
    const float rs = __builtin_amdgcn_rcpf(sc);
    float r[16];
    bool near = false;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float y = v[i] * rs;
        r[i] = __builtin_rintf(y);
        near = near || q8_near_half(y);
    }
    if (near) {
#pragma unroll
        for (int i = 0; i < 16; i++)
            if (q8_near_half(v[i] * rs)) r[i] = roundf(v[i] / sc);
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
        q[k] = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) q[k] |= (uint32_t)(uint8_t)q8_clamp(r[4 * k + i]) << (8 * i);
    }
}

CPB_DEV float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
    return v;
}

template <class T>
CPB_DEV T uniform(T v) { return (T)__builtin_amdgcn_readfirstlane((int)v); }
// a wave-uniform pointer kept in SGPRs
template <class T>
CPB_DEV T* uniform_ptr(T* p) {
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (T*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// Wave-wide maximum of a double through DPP row operations (no LDS
// round trips), returned in every lane.  Inactive / out-of-row sources read
// -inf.  Steps: quad swaps, half-row and row mirrors, then row broadcasts 15
// and 31, leaving the total in lane 63.
template <int CTRL, int ROWMASK>
CPB_DEV double dpp_max_step(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, ROWMASK, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp((int)0xFFF00000u, (int)(uint32_t)(b >> 32), CTRL, ROWMASK, 0xF, false);
    const double o = __builtin_bit_cast(double, ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
    return fmax(v, o);
}
// v from lane `src` (wave-uniform) in every lane
CPB_DEV double readlane_f64(double v, int src) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)b, src);
    const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), src);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
CPB_DEV double wave_max_f64(double v) {
    v = dpp_max_step<0xB1, 0xF>(v);     // quad_perm [1,0,3,2]
    v = dpp_max_step<0x4E, 0xF>(v);     // quad_perm [2,3,0,1]
    v = dpp_max_step<0x141, 0xF>(v);    // row_half_mirror
    v = dpp_max_step<0x140, 0xF>(v);    // row_mirror
    v = dpp_max_step<0x142, 0xA>(v);    // row_bcast:15 -> rows 1, 3
    v = dpp_max_step<0x143, 0xC>(v);    // row_bcast:31 -> rows 2, 3
    return readlane_f64(v, 63);
}

// Device-coherent access for the small buffers that workgroups hand to each
// other inside one launch (activations, routing results, hq, x).  Relaxed
// agent-scope atomics compile to plain loads/stores with the sc1 bit, which
// keep them coherent across the XCDs' separate L2s without the device-wide
// L2 writeback / invalidate that a __threadfence() costs.
template <class T>
CPB_DEV T ld_dev(const T* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
template <class T>
CPB_DEV void st_dev(T* p, T v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
// Wait until every memory operation this wave issued has completed.
// Buffer resource over [base, base + bytes).  base and bytes must be the same
// in every lane (they are made wave-uniform: lane 0's values are used); lanes
// that address different arrays need one resource over all of them.  A buffer
// load whose offset lies outside returns zeros without touching memory, so
// masked loads need no branch and the compiler waits for them by count.
CPB_DEV __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(const_cast<void*>(base)), (short)0, (int)uniform(bytes), 0x00020000);
}
// a * b for operands that fit in 24 signed bits (the k-quant block sums and
// scales): the full-rate 24-bit multiply (v_mul_i32_i24) in place of the
// quarter-rate 32-bit one; the 32-bit result is exact while |a * b| < 2^31
CPB_DEV int mul24(int a, int b) { return __mul24(a, b); }
constexpr uint32_t kOffNone = 0x80000000u;   // a buffer offset beyond every range
// 16-byte load with the cache policy of ld_dev (sc1: coherent across XCDs)
CPB_DEV u32x4 ld_dev16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 16);
}
CPB_DEV void drain_memory() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// ---- host: kernel launch with optional execution timestamps ----
// When a caller has armed a pair of events (timing mode), the next launch goes
// through hipExtLaunchKernelGGL, whose dispatch packet records them: they
// bracket that kernel's execution alone, not the queue gaps around it.
struct LaunchEvents {
    hipEvent_t start = nullptr, stop = nullptr;
};
inline LaunchEvents& armed_events() {
    static thread_local LaunchEvents ev;
    return ev;
}
template <typename F, typename... Args>
void launch(F kernel, dim3 grid, dim3 block, size_t lds, hipStream_t s, Args... args) {
    LaunchEvents& ev = armed_events();
    if (ev.start) {
        hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, s, ev.start, ev.stop, 0, args...);
        ev = LaunchEvents{};
    } else {
        hipLaunchKernelGGL(kernel, grid, block, lds, s, args...);
    }
}

// ---- LDS streaming for serial fp32 chains (sum of squares, exact router logits) ----
// The compiler's wait insertion drains every LDS read before any use inside
// the loop below; these issue eight 16-byte reads and wait for all but the
// newest eight explicitly, so one group's reads overlap the previous group's
// fma chain.  (LDS reads of a wave complete in order.)
typedef float f32x4 __attribute__((ext_vector_type(4)));
CPB_DEV uint32_t lds_addr(const float* p) {
    return (uint32_t)(size_t)(const __attribute__((address_space(3))) float*)p;
}
CPB_DEV void lds_read8(f32x4 (&o)[8], uint32_t a) {
    asm volatile(
        "ds_read_b128 %0, %8\n\t"
        "ds_read_b128 %1, %8 offset:16\n\t"
        "ds_read_b128 %2, %8 offset:32\n\t"
        "ds_read_b128 %3, %8 offset:48\n\t"
        "ds_read_b128 %4, %8 offset:64\n\t"
        "ds_read_b128 %5, %8 offset:80\n\t"
        "ds_read_b128 %6, %8 offset:96\n\t"
        "ds_read_b128 %7, %8 offset:112"
        : "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3]), "=&v"(o[4]), "=&v"(o[5]), "=&v"(o[6]), "=&v"(o[7])
        : "v"(a)
        : "memory");
}
// o (read before the newest eight LDS reads) has landed
CPB_DEV void lds_wait_older8(f32x4 (&o)[8]) {
    asm volatile("s_waitcnt lgkmcnt(8)"
                 : "+v"(o[0]), "+v"(o[1]), "+v"(o[2]), "+v"(o[3]), "+v"(o[4]), "+v"(o[5]), "+v"(o[6]), "+v"(o[7])
                 :
                 : "memory");
}
CPB_DEV void lds_wait_all() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

}  // namespace cpb
