// One instantiation unit of the MoE expert kernels per bit width: the build
// compiles this file once per K with -DEXL3_K=K.
#include "exl3_moe_impl.h"

#ifndef EXL3_K
#error "build with -DEXL3_K=<bits>"
#endif

#define EXL3_CAT2(a, b) a##b
#define EXL3_CAT(a, b) EXL3_CAT2(a, b)

namespace exl3 {
int EXL3_CAT(moe_launch_K, EXL3_K)(int cb, int ns, const MoeParams& p, hipStream_t st) {
    return moe_launch_k<EXL3_K>(cb, ns, p, st);
}
int EXL3_CAT(moe_fused_launch_K, EXL3_K)(int cb, int nsg, int nsd, const MoeParams& pg, const MoeParams& pd,
                                         hipStream_t st) {
    return moe_fused_launch_k<EXL3_K>(cb, nsg, nsd, pg, pd, st);
}
}  // namespace exl3
