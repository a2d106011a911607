// One instantiation unit of the GEMV kernels per bit width: the build
// compiles this file once per K with -DEXL3_K=K (keeps compile units small).
#include "exl3_gemv_sk.h"

#ifndef EXL3_K
#error "build with -DEXL3_K=<bits>"
#endif

#define EXL3_CAT2(a, b) a##b
#define EXL3_CAT(a, b) EXL3_CAT2(a, b)

namespace exl3 {
int EXL3_CAT(gemv_launch_K, EXL3_K)(int cb, int mb, const GemvParams& p, int experts, hipStream_t st) {
    return gemv_launch_k<EXL3_K>(cb, mb, p, experts, st);
}
int EXL3_CAT(gemv_sk_launch_K, EXL3_K)(int cb, int ns, const GemvSkParams& p, hipStream_t st) {
    return gemv_sk_launch_k<EXL3_K>(cb, ns, p, st);
}
}  // namespace exl3
