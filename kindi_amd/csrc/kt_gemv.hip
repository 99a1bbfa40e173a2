/* kt_gemv.hip - explicit instantiations of the decode product (kt_gemv.h) */
#include "kt_gemv.h"

#define KT_GINST(FMT, MT, DBG, GRP) template __global__ void k_gemv_flat<FMT, MT, DBG, GRP>(const KtGemvArgs, const KtGroupedArgs, const int8_t*, const float*, const int*, int32_t*, int);
#define KT_GINST2(FMT, MT, GRP) KT_GINST(FMT, MT, false, GRP) KT_GINST(FMT, MT, true, GRP)
KT_GINST2(0, 1, false) KT_GINST2(0, 2, false) KT_GINST2(0, 4, false)
KT_GINST2(1, 1, false) KT_GINST2(1, 2, false) KT_GINST2(1, 4, false)
KT_GINST2(1, 1, true) KT_GINST2(1, 2, true) KT_GINST2(1, 4, true)
