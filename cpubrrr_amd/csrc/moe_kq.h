// moe_kq.h -- launch arguments of the Q4_K / Q6_K (Qwen3) expert kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "moe_common.h"
#include "select.h"

namespace cpb {

// 16-byte units per superblock in the stream layouts.  Q4_K: 144 B = 9
// units.  Q6_K: ql, qh and the int8 scales (208 B = 13 units) in the unit
// stream, the fp16 d in a separate stream behind it (2 B per superblock, the
// RT rows of a (tile, superblock) contiguous), so the down stream holds
// exactly the 210 B of each superblock.  In registers the kernels keep the d
// as a 14th unit (kQ6Units).
constexpr int kQ4Units = 9;
constexpr int kQ6Units = 14;
constexpr int kQ6StreamUnits = 13;
CPB_DEV_HOST_INLINE int kq_units(int type) { return type == 12 ? kQ4Units : kQ6StreamUnits; }
CPB_DEV_HOST_INLINE int kq_sb_bytes(int type) { return type == 12 ? 144 : 210; }

// engine_qwen2.rs:40-51 converts IEEE binary16 exactly; so does the hardware.
CPB_DEV float half_bits(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

struct KqArgs {
    const u32x4* gu;         // gate+up stream layout (k_repack_kq_gateup)
    const u32x4* dn;         // down stream layout (k_repack_kq_down)
    const uint16_t* dn_d;    // Q6_K: the fp16 d stream behind dn (kq_down_dstream)
    int down_type;           // 12 (Q4_K) or 14 (Q6_K); gate/up are Q4_K
    const int8_t* xq;        // [d]   Q8_K activations
    const float* xs;         // [d/256]
    const int32_t* xsum;     // [d/32]
    const int32_t* ids;      // [top_k]  (selected by the gate/up kernel when sel.lstar is set)
    const float* wts;        // [top_k]
    SelectIn sel;            // when set, every gate/up workgroup selects at its start and workgroup 0 publishes ids / wts
    int d, dff, top_k;
    float* hbuf;             // [top_k][dff] SiLU(gate) * up
    int8_t* hq;              // [top_k][dff]      (trace only: Q8_K of hbuf)
    float* hs;               // [top_k][dff/256]  (trace only)
    int32_t* hsum;           // [top_k][dff/32]   (trace only)
    float* x;                // [d] residual, updated in place
    // trace
    float* gu_out;           // [top_k][2][dff]
    int32_t* gu_sums;        // [top_k][2][dff][d/256][2]  (sumi, mint)
    float* dn_out;           // [top_k][d]
    int32_t* dn_sums;        // [top_k][d][dff/256][nsum]  nsum = 2 (Q4_K: sumi, mint) or 1 (Q6_K)
};

// bytes of the stream layouts
size_t kq_gateup_bytes(int ne, int dff, int d);
size_t kq_down_bytes(int ne, int d, int dff, int top_k, int down_type);
// the Q6_K fp16 d stream behind the units of a down stream (null for Q4_K)
const uint16_t* kq_down_dstream(const u32x4* dn, int ne, int d, int dff, int down_type);
// re-layout from native GGUF superblock rows (device buffers, stream s)
int launch_repack_kq_gateup(const uint8_t* gate, const uint8_t* up, u32x4* out, int ne, int dff, int d, hipStream_t s);
int launch_repack_kq_down(const uint8_t* down, u32x4* out, int ne, int d, int dff, int top_k, int down_type,
                          hipStream_t s);

int launch_gateup_kq(const KqArgs& a, bool trace, hipStream_t s);
int launch_down_kq(const KqArgs& a, bool trace, hipStream_t s);

}  // namespace cpb
