/* kt_gemv_q2.hip - explicit instantiations of the decode product (kt_gemv.h): q8_0, 8 and 16 tokens */
#include "kt_gemv.h"

#define KT_INST1(FMT, MT, KS, RGB, XL) template __global__ void k_gemv<FMT, MT, KS, RGB, XL>(const KtGemvArgs, const int8_t*, const float*, const int*, int32_t*);
#define KT_INST_KR(FMT, MT, XL) KT_INST1(FMT, MT, 1, 1, XL) KT_INST1(FMT, MT, 1, 2, XL) KT_INST1(FMT, MT, 1, 4, XL) \
  KT_INST1(FMT, MT, 2, 1, XL) KT_INST1(FMT, MT, 2, 2, XL) KT_INST1(FMT, MT, 4, 1, XL) KT_INST_W8(FMT, MT, XL)
#if KT_MAXW >= 8
#define KT_INST_W8(FMT, MT, XL) KT_INST1(FMT, MT, 1, 8, XL) KT_INST1(FMT, MT, 2, 4, XL) KT_INST1(FMT, MT, 4, 2, XL)
#else
#define KT_INST_W8(FMT, MT, XL)
#endif
KT_INST_KR(1, 8, false) KT_INST_KR(1, 16, false)
