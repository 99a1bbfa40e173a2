/* kt_gemv_t1.hip - explicit instantiations of the decode product (kt_gemv.h): ternary, 1 .. 4 tokens */
#include "kt_gemv.h"

#define KT_INST1(FMT, MT, KS, RGB, XL) template __global__ void k_gemv<FMT, MT, KS, RGB, XL>(const KtGemvArgs, const int8_t*, const float*, const int*, int32_t*);
#define KT_INST_KR(FMT, MT, XL) KT_INST1(FMT, MT, 1, 1, XL) KT_INST1(FMT, MT, 1, 2, XL) KT_INST1(FMT, MT, 1, 4, XL) \
  KT_INST1(FMT, MT, 2, 1, XL) KT_INST1(FMT, MT, 2, 2, XL) KT_INST1(FMT, MT, 4, 1, XL) KT_INST_W8(FMT, MT, XL)
#if KT_MAXW >= 8
#define KT_INST_W8(FMT, MT, XL) KT_INST1(FMT, MT, 1, 8, XL) KT_INST1(FMT, MT, 2, 4, XL) KT_INST1(FMT, MT, 4, 2, XL)
#else
#define KT_INST_W8(FMT, MT, XL)
#endif
KT_INST_KR(0, 1, true) KT_INST_KR(0, 2, true) KT_INST_KR(0, 4, true)
KT_INST_KR(0, 1, false) KT_INST_KR(0, 2, false) KT_INST_KR(0, 4, false)

#define KT_PINST2(FMT, MT, KS, RPL, DBG) template __global__ void k_gemv_pipe<FMT, MT, KS, RPL, DBG>(const KtGemvArgs, const int8_t*, const float*, const int*, int32_t*);
#define KT_PINST1(FMT, MT, KS, RPL) KT_PINST2(FMT, MT, KS, RPL, false) KT_PINST2(FMT, MT, KS, RPL, true)
#define KT_PINST(FMT, MT) KT_PINST1(FMT, MT, 1, 1) KT_PINST1(FMT, MT, 1, 2) KT_PINST1(FMT, MT, 1, 4) \
  KT_PINST1(FMT, MT, 2, 1) KT_PINST1(FMT, MT, 2, 2) KT_PINST1(FMT, MT, 2, 4) KT_PINST1(FMT, MT, 4, 1) \
  KT_PINST1(FMT, MT, 4, 2) KT_PINST1(FMT, MT, 4, 4)
KT_PINST(0, 1) KT_PINST(0, 2) KT_PINST(0, 4)
