// One instantiation unit of the fat GEMM kernels per bit width: the build
// compiles this file once per K with -DEXL3_K=K.
#include "exl3_fat_impl.h"

#ifndef EXL3_K
#error "build with -DEXL3_K=<bits>"
#endif

#define EXL3_CAT2(a, b) a##b
#define EXL3_CAT(a, b) EXL3_CAT2(a, b)

namespace exl3 {
int EXL3_CAT(fat_launch_K, EXL3_K)(int cb, int mt, const FatParams& p, int splits, hipStream_t st) {
    return fat_launch_k<EXL3_K>(cb, mt, p, splits, st);
}
}  // namespace exl3
