// moe_kq.hip -- Qwen3 MoE expert GEMVs over Q4_K / Q6_K (gfx950).
#include "moe_kq.h"

namespace cpb {

int launch_gateup_kq(const KqArgs&, bool, hipStream_t) { return -22; }
int launch_down_kq(const KqArgs&, bool, hipStream_t) { return -22; }

}  // namespace cpb
