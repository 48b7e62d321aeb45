// moe_grouped.hip -- batched / prefill gpt-oss MoE layer (gfx950).
//
// Reference: the tile path engine_gpt2.rs:1120-1239, whose contract is
// "bit-identical to per-token decode" (expert-major subscriber lists, weight
// quads reused across tokens).  Here the tokens' (token, slot) pairs are
// grouped by expert and each expert's gate/up and down products run on the
// matrix cores, exactly:
//
//   v_mfma_scale_f32_32x32x64_f8f6f4, A = weights (fp4 e2m1, 32 rows x 64 K),
//   B = activations (fp8 e4m3, 64 K x 32 tokens), one MXFP4 block per
//   instruction.  A's two K halves both carry the block's 32 raw codes (the
//   16 GGUF bytes as they are: no decode), B's first half carries 16*h and the
//   second half l of each int8 activation x = 16*h + l (h = x >> 4, l in
//   [0, 15]; both exact in e4m3), and the block's e8m0 byte is A's hardware
//   scale.  Every product and partial sum is exact in fp32, so
//       D = sum_i E2M1(c_i) * x_i * 2^(e-127) = S * 2^(e-128)
//   with S the reference's int32 block sum (engine_gpt2.rs:194-228).  The
//   epilogue then does what the decode kernels do with S: per 15-block k-part
//   acc = fma(D, xsb, acc) (the same exact product S * 2^(e-128) * xsb, one
//   rounding), parts added in order, bias, SwiGLU-OAI + Q8 (gate/up) or the
//   slot-ordered combine (down).  Results are therefore the decode path's bit
//   for bit.  Blocks with e8m0 < 32 or == 255 (tbl[0] = 0 and NaN in
//   hardware, subnormal scales) are not exact this way: the caller routes
//   such layers to the per-token kernels.
//
// Operand layouts (measured on gfx950): A lane l = (row l%32, K half l/32),
// nibble n <-> K 32*half + n; B lane l = (token l%32, half hb = l/32), bytes
// 0-15 <-> K 16*hb + j, bytes 16-31 <-> K 32 + 16*hb + j; D lane l register i
// = (row 8*(i/4) + 4*(l/32) + i%4, token l%32); scale_a lane l = row l%32.
// An MXFP4 block's nibble n is element n/2 (n even) or 16 + n/2 (n odd), so
// the activation "image" of a block (64 B) puts element e's 16*h at byte
// 32*(K/16) + K%16 and its l 16 bytes later, K = 2e (e < 16) or 2(e-16)+1.
//
// The weights are read in the decode kernels' stream layout (moe_mx.hip), so
// both paths share one copy in HBM.
#include "moe_common.h"
#include "moe_grouped.h"
#include "moe_mx.h"
#include "mx_dev.h"
#include "route_dev.h"
#include "select.h"

#include <algorithm>

namespace cpb {

typedef int v8i_g __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kImg = 64;          // image bytes per 32-block


// ---- 1. per token: rmsnorm, Q8 per 32, fp8 image ----
__global__ __launch_bounds__(256) void k_prep_batch(GroupedArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int t = blockIdx.x, d = a.d, tid = threadIdx.x, nth = blockDim.x;
    float* xs = (float*)smem;
    float* xnl = xs + d;
    float* scratch = xnl + d;
    norm_into(a.x + (size_t)t * d, a.norm_w, d, a.eps, a.norm, a.norm_nt, a.apply_norm, xs, xnl, scratch);
    if (tid == 0) a.inv[t] = a.apply_norm ? scratch[16] : 1.0f;
    // Q8 per 32-block (engine_gpt2.rs:691-699), four threads per block:
    // thread c owns elements 8p + 4h .. +3 and 16 + 8p + 4h .. +3 (p = c >> 1,
    // h = c & 1), so its share of xq is two whole dwords and its share of the
    // 64-byte image two whole 8-byte runs.  Image byte K of a part (K < 16:
    // bytes 0-15, 16h; bytes 16-31, l; then the same for K 16..31 at 32-63)
    // holds element K / 2 (K even) or 16 + (K - 1) / 2 (K odd): dword w of part
    // p packs elements 8p + 2w, 8p + 2w + 16, 8p + 2w + 1, 8p + 2w + 17.  The
    // e4m3 codes come from the hardware conversion, exact for these integers;
    // the block maximum from two lane exchanges; the exact division only
    // near a rounding tie.
    for (int i = tid; i < a.nb * 4; i += nth) {
        const int bk = i >> 2, c = i & 3, p = c >> 1, h = c & 1;
        const int e0 = 8 * p + 4 * h;
        const float4 f0 = ((const float4*)(xnl + bk * 32 + e0))[0];
        const float4 f1 = ((const float4*)(xnl + bk * 32 + 16 + e0))[0];
        const float v[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
        float m = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) m = fmaxf(m, fabsf(v[k]));
        m = fmaxf(m, __shfl_xor(m, 1));
        m = fmaxf(m, __shfl_xor(m, 2));
        const float sc = fmaxf(1e-12f, m) / 127.0f;
        int q[8];
        {
            const float rs = __builtin_amdgcn_rcpf(sc);
            float r[8];
            bool near = false;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float y = v[k] * rs;
                r[k] = __builtin_rintf(y);
                near = near || q8_near_half(y);
            }
            if (near) {
#pragma unroll
                for (int k = 0; k < 8; k++)
                    if (q8_near_half(v[k] * rs)) r[k] = roundf(v[k] / sc);
            }
#pragma unroll
            for (int k = 0; k < 8; k++) q[k] = q8_clamp(r[k]);
        }
        uint32_t qw[2] = {0u, 0u};
#pragma unroll
        for (int k = 0; k < 8; k++) qw[k >> 2] |= ((uint32_t)q[k] & 0xffu) << (8 * (k & 3));
        float* xo = a.xn + (size_t)t * d + bk * 32;
        *(float4*)(xo + e0) = f0;
        *(float4*)(xo + 16 + e0) = f1;
        uint32_t* qo = (uint32_t*)(a.xq + (size_t)t * d + bk * 32);
        qo[e0 >> 2] = qw[0];
        qo[(16 + e0) >> 2] = qw[1];
        if (c == 0) a.xsb[(size_t)t * a.nb + bk] = sc;
        // elements e0 + j (k = j) and 16 + e0 + j (k = 4 + j), j < 4: dwords
        // w = 2h and 2h + 1 of part p pack (e0 + 2(w - 2h), its +16, +1, +17)
        float fh[8], fl[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int hh = q[k] >> 4;
            fh[k] = (float)(16 * hh);
            fl[k] = (float)(q[k] - 16 * hh);
        }
        uint32_t hi[2], lo[2];
#pragma unroll
        for (int w = 0; w < 2; w++) {
            const int j = 2 * w;             // elements e0 + j, 16 + e0 + j, e0 + j + 1, 16 + e0 + j + 1
            hi[w] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(fh[j + 1], fh[4 + j + 1],
                                                               __builtin_amdgcn_cvt_pk_fp8_f32(fh[j], fh[4 + j], 0, false), true);
            lo[w] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(fl[j + 1], fl[4 + j + 1],
                                                               __builtin_amdgcn_cvt_pk_fp8_f32(fl[j], fl[4 + j], 0, false), true);
        }
        uint8_t* img = a.ximg + ((size_t)t * a.nb + bk) * kImg + 32 * p + 8 * h;
        *(uint2*)img = make_uint2(hi[0], hi[1]);
        *(uint2*)(img + 16) = make_uint2(lo[0], lo[1]);
    }
}

// ---- 2. router logits, exactly: workgroup = (8 experts, 8 tokens) ----
// Every (token, expert) logit as the reference computes it
// (engine_gpt2.rs:849-852, engine_qwen2.rs:395-400): acc = b; acc += W[j] *
// xn[j] for j = 0 .. d-1, fp32, each product and each sum rounded once, in
// order.  A chain cannot be split, but a batch has n_tok * ne of them: lane
// (tl, el) of the wave runs the chain of token 8 ty + tl and expert 8 ex + el,
// the products one step ahead of the adds.  The 8 tokens' xn and the 8
// experts' router rows stream through LDS in chunks of kChainChunk (the next
// chunk requested into registers while the current one is summed).  The
// logit goes to lstar with a zero lbound: the selection then ranks exact
// values and never needs its exact path, and the weights are the softmax of
// the reference's own fp32 logits.
constexpr int kChainChunk = 128;
constexpr int kChainStride = kChainChunk + 4;     // floats per LDS row (spreads the 8 rows over the banks)
__global__ __launch_bounds__(64) void k_router_exact(GroupedArgs a) {
    __shared__ __align__(16) float xs[2][8][kChainStride];
    __shared__ __align__(16) float wsh[2][8][kChainStride];
    const int lane = threadIdx.x, d = a.d;
    const int tl = lane >> 3, el = lane & 7;
    const int t = blockIdx.y * 8 + tl, e = blockIdx.x * 8 + el;
    // staging: lane moves 16-byte pieces c = lane + 64 i (i < 4) of the
    // 8 x 128-float chunk: row c / 32, floats 4 (c % 32) ..
    const int nt = a.n_tok, ne = a.ne;
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(a.xn, (uint32_t)((size_t)nt * d * 4));
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(a.router_w, (uint32_t)((size_t)ne * d * 4));
    auto fetch = [&](int j0, u32x4 (&xr)[4], u32x4 (&wr)[4]) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = lane + 64 * i, row = c >> 5, j = j0 + 4 * (c & 31);
            const int tt = blockIdx.y * 8 + row, ee = blockIdx.x * 8 + row;
            xr[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, tt < nt && j < d ? (uint32_t)(((size_t)tt * d + j) * 4) : kOffNone, 0, 0);
            wr[i] = __builtin_amdgcn_raw_buffer_load_b128(rw, ee < ne && j < d ? (uint32_t)(((size_t)ee * d + j) * 4) : kOffNone, 0, 0);
        }
    };
    auto put = [&](int buf, const u32x4 (&xr)[4], const u32x4 (&wr)[4]) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = lane + 64 * i, row = c >> 5, f = 4 * (c & 31);
            *(u32x4*)&xs[buf][row][f] = xr[i];
            *(u32x4*)&wsh[buf][row][f] = wr[i];
        }
    };
    float acc = (a.router_b && e < ne) ? a.router_b[e] : 0.0f;
    u32x4 xr[4], wr[4];
    fetch(0, xr, wr);
    put(0, xr, wr);
    const int nch = (d + kChainChunk - 1) / kChainChunk;
    for (int ch = 0; ch < nch; ch++) {
        const int buf = ch & 1;
        if (ch + 1 < nch) fetch((ch + 1) * kChainChunk, xr, wr);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int n = min(kChainChunk, d - ch * kChainChunk);   // a multiple of 32 (d % 32 == 0)
        const float* xp = &xs[buf][tl][0];
        const float* wp = &wsh[buf][el][0];
        for (int j = 0; j < n; j += 32) {
            f32x4 xv[8], wv[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                xv[u] = *(const f32x4*)(xp + j + 4 * u);
                wv[u] = *(const f32x4*)(wp + j + 4 * u);
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
#pragma unroll
                for (int c = 0; c < 4; c++) acc = __fadd_rn(acc, __fmul_rn(wv[u][c], xv[u][c]));
            }
        }
        if (ch + 1 < nch) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            put(buf ^ 1, xr, wr);
        }
    }
    if (t < nt && e < ne) {
        a.lstar[(size_t)t * ne + e] = (double)acc;
        a.lbound[(size_t)t * ne + e] = 0.0;
    }
}


// ---- 3. top-k + softmax, one wavefront per token (the decode kernels'
// selection code; on the exact logits of k_router_exact its intervals are
// points, so the ids are the reference's and the weights the softmax of the
// reference's fp32 logits) ----
__global__ __launch_bounds__(64) void k_select_batch(GroupedArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ Selection sel;
    const int lane = threadIdx.x, t = blockIdx.x;
    SelectIn si{};
    si.lstar = a.lstar + (size_t)t * a.ne;
    si.lbound = a.lbound + (size_t)t * a.ne;
    si.router_w = a.router_w;
    si.router_b = a.router_b;
    si.xn = a.xn + (size_t)t * a.d;
    si.ne = a.ne; si.k = a.k; si.d = a.d;
    si.logits = a.logits + (size_t)t * a.ne;      // written by every workgroup: one per token
    select_topk_wave<8, 4>(si, smem, &sel, true);
    if (lane < a.k) {
        const int e = sel.ids[lane];
        a.ids[(size_t)t * a.k + lane] = e;
        a.wts[(size_t)t * a.k + lane] = sel.wts[lane];
    }
    if (lane == 0) a.fallback[t] = sel.fallback;
}

// ---- 4. grouping by expert ----
// One workgroup: each pair takes its place among its expert's pairs from an
// LDS counter (arrival order: any order serves, a pair's outputs do not
// depend on its tile or on the other pairs there), then the exclusive prefix
// of the counts (pairs and 32-pair tiles), each pair written at its expert's
// offset + its place, and the tile list.
constexpr int kScanPer = 16;                   // pairs per thread held in registers
// One workgroup; the caller's config check bounds n_expert <= 256 (the LDS
// tables) and n_tok * k <= 16384 = kScanPer * 1024 (the pairs per thread).
__global__ __launch_bounds__(1024) void k_group_scan(GroupedArgs a) {
    __shared__ int cnt_l[256], off_l[256], toff_l[256];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int np = a.n_tok * a.k, ne = a.ne;
    for (int e = tid; e < ne; e += blockDim.x) cnt_l[e] = 0;
    // every pair's expert requested before the first wait
    int ex[kScanPer], rk[kScanPer];
#pragma unroll
    for (int u = 0; u < kScanPer; u++) {
        const int p = tid + u * 1024;
        ex[u] = p < np ? a.ids[p] : -1;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kScanPer; u++)
        rk[u] = ex[u] >= 0 ? __hip_atomic_fetch_add(cnt_l + ex[u], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) : 0;
    __syncthreads();
    if (w == 0) {
        int o = 0, to = 0;
        for (int base = 0; base < ne; base += 64) {
            const int e = base + lane;
            const int c = e < ne ? cnt_l[e] : 0;
            const int tl = (c + 31) / 32;
            int ic = c, it = tl;
#pragma unroll
            for (int s2 = 1; s2 < 64; s2 <<= 1) {
                const int uc = __shfl_up(ic, s2), ut = __shfl_up(it, s2);
                if (lane >= s2) { ic += uc; it += ut; }
            }
            if (e < ne) { off_l[e] = o + ic - c; toff_l[e] = to + it - tl; }
            o += __shfl(ic, 63);
            to += __shfl(it, 63);
        }
        if (lane == 0) *a.ntiles = to;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kScanPer; u++)
        if (ex[u] >= 0) a.sorted[off_l[ex[u]] + rk[u]] = tid + u * 1024;
    for (int e = w; e < ne; e += 16) {
        const int c = cnt_l[e], nt = (c + 31) / 32;
        for (int j = lane; j < nt; j += 64) a.tiles[toff_l[e] + j] = int4{e, off_l[e] + 32 * j, min(32, c - 32 * j), 0};
    }
}

// One block of the grouped product: A = 16 raw code bytes (both K halves),
// B = the 32-byte half-image, hardware scale = the block's e8m0 byte.
// SEL: which byte of the word ew is the block's e8m0 (the instruction's
// scale operand select), so four blocks share one scale register
template <int SEL>
CPB_DEV v16f mx_block_mfma(const u32x4& w, const u32x4& x0, const u32x4& x1, uint32_t ew) {
    const v8i_g A = {(int)w[0], (int)w[1], (int)w[2], (int)w[3], 0, 0, 0, 0};
    const v8i_g B = {(int)x0[0], (int)x0[1], (int)x0[2], (int)x0[3], (int)x1[0], (int)x1[1], (int)x1[2], (int)x1[3]};
    const v16f Z = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(A, B, Z, 4, 0, SEL, (int)ew, 0, 127);
}
// the same with the byte index a value that is constant once the caller's
// loop is unrolled
CPB_DEV v16f mx_block_mfma_b(const u32x4& w, const u32x4& x0, const u32x4& x1, uint32_t ew, int sel) {
    switch (sel & 3) {
        case 0: return mx_block_mfma<0>(w, x0, x1, ew);
        case 1: return mx_block_mfma<1>(w, x0, x1, ew);
        case 2: return mx_block_mfma<2>(w, x0, x1, ew);
        default: return mx_block_mfma<3>(w, x0, x1, ew);
    }
}

// LDS staging of one k-part's activations for a 32-token tile: per block i
// and token ti a 64-byte slot whose four 16-byte chunks are XOR-swizzled by
// the token (chunk c at position c ^ swz(ti)), then room for 512 scales (15 x
// 32 used).  The swizzle puts the reads (lane ti reads chunk 2hb or 2hb + 1 of
// slot ti) on distinct banks in every group of 8 and of 16 lanes (80-byte
// padded slots had 2.75 M conflict cycles per gate/up launch).
constexpr int kSlot = 64;
constexpr int kStageBlk = 15;
constexpr int kStageBytes = kStageBlk * 32 * kSlot + 512 * 4;
CPB_DEV_HOST_INLINE int stage_swz(int ti) { return ((ti >> 1) ^ (ti >> 2)) & 3; }

// Workgroup sizes of the grouped GEMMs.  Gate/up: 4 waves, so that two
// workgroups share a CU (LDS 2 x 65 KB, <= 256 registers per lane) and one's
// barriers, prologue and SwiGLU epilogue overlap the other's k-part loop.
// Down (a short epilogue): 8 waves, whose row tiles share one staged
// activation tile.
constexpr int kGuThreads = 256, kDnThreads = 512;


// Direct global-to-LDS staging of k-part q (no staging registers): each
// wavefront instruction writes 1 KB of LDS, lane L at byte 16 L, so lane L
// fetches the chunk the swizzled layout puts there (token h*16 + L/4 of the
// block, chunk (L & 3) ^ swz(token)); the scales take 8 instructions of 64
// (the last half past block 14 reads nothing).
typedef __attribute__((address_space(3))) void lds_void_g;
struct DmaPlan {
    __amdgpu_buffer_rsrc_t ri, rs;
    uint32_t vbase0, vbase1, sbase;  // bytes: block 0 of the lane's chunk in token half 0 / 1, its scale
};
CPB_DEV DmaPlan dma_plan(const uint8_t* img, const float* sc, size_t rows, int nbk, const int* src) {
    const int L = threadIdx.x & 63;
    DmaPlan p;
    p.ri = buf_rsrc(img, (uint32_t)(rows * nbk * kImg));
    p.rs = buf_rsrc(sc, (uint32_t)(rows * nbk * 4));
    const int t0 = L >> 2, t1 = 16 + (L >> 2), r0 = src[t0], r1 = src[t1];
    p.vbase0 = r0 >= 0 ? (uint32_t)r0 * nbk * kImg + (uint32_t)(((L & 3) ^ stage_swz(t0)) << 4) : kOffNone;
    p.vbase1 = r1 >= 0 ? (uint32_t)r1 * nbk * kImg + (uint32_t)(((L & 3) ^ stage_swz(t1)) << 4) : kOffNone;
    const int rs_ = src[L & 31];
    p.sbase = rs_ >= 0 ? (uint32_t)rs_ * nbk * 4 : kOffNone;
    return p;
}
template <int NT>
CPB_DEV void stage_dma(const DmaPlan& p, int nbk, int q, unsigned char* st) {
    // the wave index as a scalar: every condition and LDS address below is
    // then scalar work
    const int w = uniform((int)(threadIdx.x >> 6)), L = threadIdx.x & 63;
    const int lim = min(kBlkPerPart, nbk - q * kBlkPerPart);
#pragma unroll
    for (int k = 0; k < (2 * kBlkPerPart + NT / 64 - 1) / (NT / 64); k++) {
        const int m = w + k * (NT / 64), i = m >> 1, h = m & 1;
        if (m < 2 * kBlkPerPart) {
            const uint32_t off = i < lim ? (h ? p.vbase1 : p.vbase0) + (uint32_t)(q * kBlkPerPart + i) * kImg : kOffNone;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(p.ri, (lds_void_g*)(st + (i * 32 + h * 16) * kSlot), 16, off, 0, 0, 0);
        }
    }
#pragma unroll
    for (int k = 0; k < (8 + NT / 64 - 1) / (NT / 64); k++) {
        const int n = w + k * (NT / 64), i = 2 * n + (L >> 5);
        if (n < 8) {
            const uint32_t off = i < lim ? p.sbase + (uint32_t)(q * kBlkPerPart + i) * 4 : kOffNone;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(p.rs, (lds_void_g*)(st + kStageBlk * 32 * kSlot + n * 256), 4, off, 0, 0, 0);
        }
    }
}
// the two staging buffers of the DMA-staged GEMMs, as separate objects so
// that the compiler can tell the buffer being filled from the one being read
__shared__ __align__(16) unsigned char g_stage0[kStageBytes];
__shared__ __align__(16) unsigned char g_stage1[kStageBytes];

// Weight operand of one k-part for the lane's row: unit u (0 = the e8m0
// bytes, 1..15 = blocks) sits at byte off + u * ustride of the expert's
// stream; rs covers the expert's whole stream (out-of-range offsets read 0).
struct WeightStream {
    __amdgpu_buffer_rsrc_t rs;
    uint32_t off, ustride, pstride;      // bytes: lane's unit 0 of k-part 0, unit step, k-part step
};
CPB_DEV u32x4 wload(const WeightStream& ws, int q, int u) {
    return __builtin_amdgcn_raw_buffer_load_b128(ws.rs, ws.off + (uint32_t)q * ws.pstride + (uint32_t)u * ws.ustride, 0, 0);
}

// The k-part loop shared by the two grouped GEMMs.  Per k-part, D = A(rows)
// x B(tokens) per block on the matrix cores and acc = fma(D, xsb, acc) in
// block order, in two chains (blocks 0-7 and 8-14, as the decode kernels'
// two wavefronts per k-part), the chains added to the total in order.
//
// Software pipeline: block i + 1's MFMA is issued before block i's sixteen
// fmas (two D register sets), so the matrix core and the VALU run side by
// side; each weight register is refilled with the next k-part's unit right
// after its MFMA has been issued (one k-part of lead time, 16 units of
// registers instead of 32).  Two LDS staging buffers alternate for the
// activations: right after the barrier that opens k-part q, the direct loads
// of k-part q + 1 go into the other buffer (every wave has finished reading it
// in k-part q - 1), so one barrier per k-part suffices; the barrier's release
// fence makes each wave wait for its own direct loads first.
// TRACE writes the int32 block sums S = D * 2^(128 - e) of valid rows.
template <bool TRACE, int NT>
CPB_DEV v16f grouped_parts(const WeightStream& ws, int P, const uint8_t* img, const float* sc,
                           size_t rows, int nbk, const int* src, int lane, int32_t* tb, bool trace_ok,
                           float* bias_lds, float bias_v, int nbias) {
    const int ti = lane & 31, hb = lane >> 5;
    // the lane's two 16-byte chunks (2hb, 2hb + 1) of its token's slot
    const int o0 = ((2 * hb) ^ stage_swz(ti)) << 4, o1 = ((2 * hb + 1) ^ stage_swz(ti)) << 4;
    u32x4 wv[kUnits];
#pragma unroll
    for (int u = 0; u < kUnits; u++) wv[u] = wload(ws, 0, u);
    const DmaPlan dp = dma_plan(img, sc, rows, nbk, src);
    stage_dma<NT>(dp, nbk, 0, g_stage0);
    v16f tot = {};
    // k-part q on the activations staged in st; the next k-part's go to nx
    auto kpart = [&](int q, unsigned char* st, unsigned char* nx) {
        __syncthreads();                     // k-part q's activations have landed
        // past the last k-part the refills read out of range (zeros, no traffic)
        const int qn = q + 1 < P ? q + 1 : 0x7fff;
        const u32x4 ex = wv[0];
        wv[0] = wload(ws, qn, 0);
        if (q + 1 < P) stage_dma<NT>(dp, nbk, q + 1, nx);
        const unsigned char* xp = st + ti * kSlot;
        const float* sl = (const float*)(st + kStageBlk * 32 * kSlot) + ti;
        v16f acc = {}, Dc, Dn;
        float sc_c, sc_n;
        // activation operands two blocks ahead: buffer j & 1 holds block j's
        // until its MFMA is issued, then takes block j + 2's
        u32x4 xa[2][2];
        float sa[2];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            xa[j][0] = *(const u32x4*)(xp + j * 32 * kSlot + o0);
            xa[j][1] = *(const u32x4*)(xp + j * 32 * kSlot + o1);
            sa[j] = sl[j * 32];
        }
        {
            sc_c = sa[0];
            Dc = mx_block_mfma<0>(wv[1], xa[0][0], xa[0][1], ex[0]);
            wv[1] = wload(ws, qn, 1);
            xa[0][0] = *(const u32x4*)(xp + 2 * 32 * kSlot + o0);
            xa[0][1] = *(const u32x4*)(xp + 2 * 32 * kSlot + o1);
            sa[0] = sl[2 * 32];
        }
#pragma unroll
        for (int i = 0; i < kBlkPerPart; i++) {
            if (i + 1 < kBlkPerPart) {
                const int j = i + 1, bj = j & 1;
                sc_n = sa[bj];
                Dn = mx_block_mfma_b(wv[1 + j], xa[bj][0], xa[bj][1], ex[j >> 2], j);
                wv[1 + j] = wload(ws, qn, 1 + j);
                if (j + 2 < kBlkPerPart) {
                    xa[bj][0] = *(const u32x4*)(xp + (j + 2) * 32 * kSlot + o0);
                    xa[bj][1] = *(const u32x4*)(xp + (j + 2) * 32 * kSlot + o1);
                    sa[bj] = sl[(j + 2) * 32];
                }
            }
            // keep the order as written (the scheduler would sink the reads
            // next to their MFMA)
            __builtin_amdgcn_sched_barrier(0);
            if (TRACE) {
                const int b = q * kBlkPerPart + i;
                const uint32_t eb = (ex[i >> 2] >> (8 * (i & 3))) & 0xffu;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int rl = 8 * (r >> 2) + 4 * hb + (r & 3);
                    const int e_r = __shfl((int)eb, rl);
                    if (trace_ok && b < nbk) tb[rl * (size_t)nbk + b] = (int)ldexpf(Dc[r], 128 - e_r);
                }
            }
#pragma unroll
            for (int r = 0; r < 16; r++) acc[r] = fmaf(Dc[r], sc_c, acc[r]);
            if (i == kSubUnits - 1 || i == kBlkPerPart - 1) {
                // end of a chain: into the total, in order
#pragma unroll
                for (int r = 0; r < 16; r++) tot[r] += acc[r];
                acc = v16f{};
            }
            Dc = Dn;
            sc_c = sc_n;
        }
    };
    for (int q = 0; q < P; q++) kpart(q, (q & 1) ? g_stage1 : g_stage0, (q & 1) ? g_stage0 : g_stage1);
    // the caller's bias, loaded at its start, into LDS for its epilogue
    if (threadIdx.x < nbias) bias_lds[threadIdx.x] = bias_v;
    __syncthreads();             // callers reuse the LDS
    return tot;
}

// ---- 5. grouped gate/up + SwiGLU-OAI + Q8 (+ image of h) ----
// one workgroup per (token tile, group of 2 row tiles) (grouped_item); 4
// waves: wave w = row tile w/2 of the group, gate (w even) or up (w odd).
template <bool TRACE>
__global__ __launch_bounds__(kGuThreads) __attribute__((amdgpu_waves_per_eu(2))) void k_gateup_grouped(GroupedArgs a) {
    __shared__ int src[32];
    const int T = a.dff / 32, P = a.parts_gu, nb = a.nb;
    int tile, grp;
    if (!grouped_item(uniform(*a.ntiles), (T + 1) / 2, &tile, &grp)) return;
    const int4 tl = a.tiles[tile];
    const int e = uniform(tl.x), start = uniform(tl.y), cnt = uniform(tl.z);
    const int lane = threadIdx.x & 63, w = uniform((int)(threadIdx.x >> 6));
    const int rt = grp * 2 + (w >> 1), isup = w & 1;
    const bool live = rt < T;
    if (threadIdx.x < 32) src[threadIdx.x] = (int)threadIdx.x < cnt ? a.sorted[start + threadIdx.x] / a.k : -1;
    __syncthreads();
    // the biases of the workgroup's 2 x (32 gate + 32 up) rows, requested now
    // and kept in one register until the epilogue (a load issued after the
    // GEMM would wait a full loaded-memory latency)
    __shared__ float bias_s[128];                   // [row tile][gate 32 | up 32]
    float bias_v = 0.0f;
    {
        const int t = (int)threadIdx.x, rtb = grp * 2 + (t >> 6), gu = (t >> 5) & 1;
        const float* bp = gu ? a.up_b : a.gate_b;
        if (t < 128 && bp && rtb < T) bias_v = bp[(size_t)e * a.dff + rtb * 32 + (t & 31)];
    }
    const int ti = lane & 31, hb = lane >> 5;
    const bool valid = ti < cnt;
    const int pair = valid ? a.sorted[start + ti] : 0;
    WeightStream ws;
    {
        const size_t ex_units = (size_t)T * P * kUnits * 64;         // one expert's gate/up stream
        ws.rs = buf_rsrc(a.gu + (size_t)e * ex_units, (uint32_t)(ex_units * 16));
        ws.off = (uint32_t)((((size_t)(live ? rt : T) * P) * kUnits * 64 + isup * 32 + (lane & 31)) * 16);
        ws.ustride = 64 * 16;
        ws.pstride = kUnits * 64 * 16;
    }
    int32_t* tb = TRACE ? a.gu_sums + (((size_t)pair * 2 + isup) * a.dff + rt * 32) * nb : nullptr;

    const v16f tot = grouped_parts<TRACE, kGuThreads>(ws, P, a.ximg, a.xsb, (size_t)a.n_tok, nb, src, lane, tb,
                                          valid && live, bias_s, bias_v, 128);
    // SwiGLU, Q8 and image of the row tile, split over its two waves: the
    // lane's rows 8g + 4hb + c (g, c < 4) of groups g = isup and g = isup + 2
    // are this wave's (so each wave owns whole hq words and whole 8-byte image
    // runs); each wave hands the partner the totals of the partner's rows
    // (LDS reused), then the block maximum is combined through LDS.
    const int rtl = w >> 1;
    float* xch = (float*)g_stage0;                // [row tile][sender][8][64]
    float* mxs = xch + 2 * 2 * 8 * 64;            // [row tile][wave][64]
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int r = 4 * (1 - isup) + (j & 3) + 8 * (j >> 2);        // partner's j-th row
        xch[((rtl * 2 + isup) * 8 + j) * 64 + lane] = tot[r];
    }
    __syncthreads();
    float hv[8], m = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int r = 4 * isup + (j & 3) + 8 * (j >> 2);                // this wave's j-th row
        const int rr = 8 * (r >> 2) + 4 * hb + (r & 3);                 // row within the tile
        const float own = tot[r], oth = xch[((rtl * 2 + 1 - isup) * 8 + j) * 64 + lane];
        float vg = isup ? oth : own, vu = isup ? own : oth;
        if (a.gate_b) vg += bias_s[rtl * 64 + rr];
        if (a.up_b) vu += bias_s[rtl * 64 + 32 + rr];
        const float xg = fminf(vg, a.limit);                           // engine_gpt2.rs:887-906
        const float yu = fminf(fmaxf(vu, -a.limit), a.limit);
        hv[j] = (xg / (1.0f + expf(-a.alpha * xg))) * (yu + 1.0f);
        m = fmaxf(m, fabsf(hv[j]));
    }
    m = fmaxf(m, __shfl_xor(m, 32));
    mxs[(rtl * 2 + isup) * 64 + lane] = m;
    __syncthreads();
    m = fmaxf(m, mxs[(rtl * 2 + 1 - isup) * 64 + lane]);
    const float sc = fmaxf(1e-12f, m) / 127.0f;
    if (!valid || !live) return;
    // hq: the lane's groups g = isup, isup + 2 as 4-byte words; image: elements
    // e and e + 16 sit at adjacent K (2e, 2e + 1), so groups g and g + 2 fill
    // the 8 bytes K = 16 isup + 8hb .. +7 of each half
    uint8_t* img = a.himg + ((size_t)pair * a.nbf + rt) * kImg;
    // Q8 of the 8 values (the exact division only when some lane's quotient
    // lies near a rounding tie), then the bytes: qw[gh] byte c = value
    // j = 4 gh + c; the image run's byte 2 (c & 1) + gh of word c >> 1 holds
    // value j's 16h (hi) and l (lo) as e4m3, whose hardware conversion is
    // exact for these integers (|16h| <= 128, 0 <= l <= 15)
    int qv[8];
    {
        const float rs = __builtin_amdgcn_rcpf(sc);
        float r[8];
        bool near = false;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float y = hv[j] * rs;
            r[j] = __builtin_rintf(y);
            near = near || q8_near_half(y);
        }
        if (near) {
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (q8_near_half(hv[j] * rs)) r[j] = roundf(hv[j] / sc);
        }
#pragma unroll
        for (int j = 0; j < 8; j++) qv[j] = q8_clamp(r[j]);
    }
    uint32_t qw[2] = {0u, 0u}, hi[2], lo[2];
#pragma unroll
    for (int j = 0; j < 8; j++) qw[j >> 2] |= ((uint32_t)qv[j] & 0xffu) << (8 * (j & 3));
    float fh[8], fl[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int h = qv[j] >> 4;
        fh[j] = (float)(16 * h);
        fl[j] = (float)(qv[j] - 16 * h);
    }
#pragma unroll
    for (int w2 = 0; w2 < 2; w2++) {
        // word w2: bytes (c = 2 w2, gh 0), (c = 2 w2, gh 1), (c = 2 w2 + 1, gh 0), (c = 2 w2 + 1, gh 1)
        const int c0 = 2 * w2, c1 = 2 * w2 + 1;
        hi[w2] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(fh[c1], fh[4 + c1],
                                                            __builtin_amdgcn_cvt_pk_fp8_f32(fh[c0], fh[4 + c0], 0, false), true);
        lo[w2] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(fl[c1], fl[4 + c1],
                                                            __builtin_amdgcn_cvt_pk_fp8_f32(fl[c0], fl[4 + c0], 0, false), true);
    }
    uint32_t* hqw = (uint32_t*)(a.hq + (size_t)pair * a.dff + rt * 32 + 8 * isup + 4 * hb);
    hqw[0] = qw[0];
    hqw[4] = qw[1];
    *(uint2*)(img + 32 * isup + 8 * hb) = make_uint2(hi[0], hi[1]);
    *(uint2*)(img + 32 * isup + 8 * hb + 16) = make_uint2(lo[0], lo[1]);
    if (hb == 0 && !isup) a.hsb[(size_t)pair * a.nbf + rt] = sc;
}

// ---- 6. grouped down (+ bias) into dnout ----
// one workgroup per (token tile, group of 8 row tiles of 32 rows) (grouped_item).
template <bool TRACE>
__global__ __launch_bounds__(kDnThreads) void k_down_grouped(GroupedArgs a) {
    __shared__ int src[32];
    int tile, grp;
    if (!grouped_item(uniform(*a.ntiles), (a.d / 32 + 7) / 8, &tile, &grp)) return;
    const int4 tl = a.tiles[tile];
    const int e = uniform(tl.x), start = uniform(tl.y), cnt = uniform(tl.z);
    const int lane = threadIdx.x & 63, w = uniform((int)(threadIdx.x >> 6));
    const int RTv = mx_down_rt(a.k), Tv = a.d / RTv, P = a.parts_dn, nbf = a.nbf;
    const int rt = grp * 8 + w;
    const bool live = rt < a.d / 32;
    if (threadIdx.x < 32) src[threadIdx.x] = (int)threadIdx.x < cnt ? a.sorted[start + threadIdx.x] : -1;
    __syncthreads();
    const int ti = lane & 31, hb = lane >> 5;
    const bool valid = ti < cnt;
    const int pair = valid ? a.sorted[start + ti] : 0;
    const int row_l = rt * 32 + (lane & 31);                          // this lane's A row
    // the biases of the workgroup's 8 x 32 rows, requested now (one register
    // until the epilogue)
    __shared__ float bias_s[256];
    float bias_v = 0.0f;
    if (threadIdx.x < 256 && a.down_b && grp * 256 + (int)threadIdx.x < a.d)
        bias_v = a.down_b[(size_t)e * a.d + grp * 256 + threadIdx.x];
    WeightStream ws;
    {
        const size_t ex_units = (size_t)Tv * P * kUnits * RTv;      // one expert's down stream
        ws.rs = buf_rsrc(a.dn + (size_t)e * ex_units, (uint32_t)(ex_units * 16));
        ws.off = live ? (uint32_t)(((size_t)(row_l / RTv) * P * kUnits * RTv + row_l % RTv) * 16) : kOffNone;
        ws.ustride = RTv * 16;
        ws.pstride = kUnits * RTv * 16;
    }
    int32_t* tb = TRACE ? a.dn_sums + ((size_t)pair * a.d + rt * 32) * nbf : nullptr;

    const v16f tot = grouped_parts<TRACE, kDnThreads>(ws, P, a.himg, a.hsb, (size_t)a.n_tok * a.k, nbf, src, lane,
                                          tb, valid && live, bias_s, bias_v, 256);
    if (!valid || !live) return;
    float* out = a.dnout + (size_t)pair * a.d + rt * 32 + 4 * hb;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        float4 v;
        float* vp = (float*)&v;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int row = rt * 32 + 8 * g + 4 * hb + c;
            vp[c] = tot[4 * g + c] + (a.down_b ? bias_s[row - grp * 256] : 0.0f);
        }
        *(float4*)(out + 8 * g) = v;
    }
}

// ---- 7. per token: x += sum over slots (ascending) of wts * (down + bias) ----
// one thread per 4 consecutive elements (d % 4 == 0), the same fp32 operations
// in the same order as a scalar loop
__global__ __launch_bounds__(256) void k_combine_batch(GroupedArgs a) {
    const int d4 = a.d / 4, K = a.k;
    const size_t n4 = (size_t)a.n_tok * d4;
    const float4* __restrict__ dn = (const float4*)a.dnout;
    float4* __restrict__ x = (float4*)a.x;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n4; i += (size_t)gridDim.x * blockDim.x) {
        const size_t t = i / d4, r4 = i % d4;
        float4 v[8];
        float wk[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            v[k] = k < K ? dn[(t * K + k) * d4 + r4] : float4{0, 0, 0, 0};
            wk[k] = k < K ? a.wts[t * K + k] : 0.0f;
        }
        float4 s = x[i];                                     // engine_gpt2.rs:911-921
#pragma unroll
        for (int k = 0; k < 8; k++) {
            if (k < K) {
                s.x += wk[k] * v[k].x;
                s.y += wk[k] * v[k].y;
                s.z += wk[k] * v[k].z;
                s.w += wk[k] * v[k].w;
            }
        }
        x[i] = s;
    }
}

int launch_grouped_layer(const GroupedArgs& a, bool trace, hipStream_t s, const LaunchEvents* ev) {
    const int nt = a.n_tok;
    if (a.kq) {
        if (launch_prep_kq(a, s)) return -19;
    } else {
        launch(k_prep_batch, dim3(nt), dim3(256), sizeof(float) * (2 * a.d + 64), s, a);
    }
    // one thread per kRouteC elements, whole waves (the decode route's element waves)
    launch(k_router_exact, dim3((a.ne + 7) / 8, (nt + 7) / 8), dim3(64), 0, s, a);
    launch(k_select_batch, dim3(nt), dim3(64), select_lds_bytes(a.ne, a.d, kExactGroupWide), s, a);
    launch(k_group_scan, dim3(1), dim3(1024), 0, s, a);
    if (a.kq) {
        if (launch_kq_gemms(a, trace, s, ev)) return -19;
        launch(k_combine_batch, dim3((unsigned)std::min<size_t>(((size_t)nt * (a.d / 4) + 255) / 256, 2048)), dim3(256), 0, s, a);
        return hipGetLastError() == hipSuccess ? 0 : -19;
    }
    // one workgroup per (token tile, row group), dealt out by grouped_item:
    // 8 slots per XCD round, enough for the largest tile count
    const int ngu = a.max_tiles * ((a.dff / 32 + 1) / 2), ndn = a.max_tiles * ((a.d / 32 + 7) / 8);
    const dim3 ggu((ngu + 7) / 8 * 8), gdn((ndn + 7) / 8 * 8);
    if (ev) armed_events() = ev[0];
    if (trace) launch(k_gateup_grouped<true>, ggu, dim3(kGuThreads), 0, s, a);
    else launch(k_gateup_grouped<false>, ggu, dim3(kGuThreads), 0, s, a);
    if (ev) armed_events() = ev[1];
    if (trace) launch(k_down_grouped<true>, gdn, dim3(kDnThreads), 0, s, a);
    else launch(k_down_grouped<false>, gdn, dim3(kDnThreads), 0, s, a);
    launch(k_combine_batch, dim3((unsigned)std::min<size_t>(((size_t)nt * (a.d / 4) + 255) / 256, 2048)), dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -19;
}

}  // namespace cpb
