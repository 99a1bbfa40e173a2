/* kt_gemv.hip - explicit instantiations of the decode product (kt_gemv.h) */
#include "kt_gemv.h"

#define KT_GINST(FMT, MT, DBG) template __global__ void k_gemv_flat<FMT, MT, DBG>(const KtGemvArgs, const int8_t*, const float*, const int*, int32_t*, int);
#define KT_GINST2(FMT, MT) KT_GINST(FMT, MT, false) KT_GINST(FMT, MT, true)
KT_GINST2(0, 1) KT_GINST2(0, 2) KT_GINST2(0, 4)
KT_GINST2(1, 1) KT_GINST2(1, 2) KT_GINST2(1, 4)
