/* kt_gemv.hip - explicit instantiations of the decode product (kt_gemv.h) */
#include "kt_gemv.h"

/* one token a chunk: k_gemv_flat1 (64 VGPRs); 2 and 4 tokens a chunk: k_gemv_flat */
#define KT_GINST(K, FMT, MT, DBG, GRP) template __global__ void K<FMT, MT, DBG, GRP>(const KtGemvArgs, const KtGroupedArgs, const int8_t*, const float*, const int*, int32_t*, int);
#define KT_GINST2(K, FMT, MT, GRP) KT_GINST(K, FMT, MT, false, GRP) KT_GINST(K, FMT, MT, true, GRP)
KT_GINST2(k_gemv_flat1, 0, 1, false) KT_GINST2(k_gemv_flat, 0, 2, false) KT_GINST2(k_gemv_flat, 0, 4, false)
KT_GINST2(k_gemv_flat1, 1, 1, false) KT_GINST2(k_gemv_flat, 1, 2, false) KT_GINST2(k_gemv_flat, 1, 4, false)
KT_GINST2(k_gemv_flat1, 1, 1, true) KT_GINST2(k_gemv_flat, 1, 2, true) KT_GINST2(k_gemv_flat, 1, 4, true)
/* q8_0 grouped products with their activations quantized in the staging (up: plain; down: relu^2 first) */
KT_GINST(k_gemv_flat1, 2, 1, false, true) KT_GINST(k_gemv_flat, 2, 2, false, true)
KT_GINST(k_gemv_flat1, 3, 1, false, true) KT_GINST(k_gemv_flat, 3, 2, false, true)

#ifdef KT_TRACE
extern "C" int kt_trace_gemv_read(void* host){
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(kt_trace_buf), sizeof(kt_trace_buf), 0, hipMemcpyDeviceToHost);
}
extern "C" int kt_trace_gemv_enable(int on){
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(kt_trace_on), &on, sizeof(int), 0, hipMemcpyHostToDevice);
}
#endif
