/* kt_topk.h - the router's top-k by one wave, shared by the MoE dispatch kernels (kt_moe.hip) and the one-token MoE
   chain (kt_moe1.hip). Two scorings (KtRouter.score):
   KT_SCORE_SOFTMAX: softmax over E logits, the k largest, weights normalised over the chosen k.
     The selection compares logits (the softmax is monotone; ties to the lower expert index) and the weights are
     exp(l_j - l_max) / sum over the chosen of exp(l_i - l_max): the full softmax denominator cancels.
   KT_SCORE_SIGMOID (Kindi's Lightning router, lt_topk / lt_router_topk lightning.cu:373-468): s_e = 1 / (1 +
     exp(-l_e)), the k largest of s_e + bias[e] (ties to the lower expert index), weights s_j / (sum over the chosen s,
     in pick order) * scale. */
#pragma once
#include "kt_common.h"

#define KT_SCORE_SOFTMAX 0
#define KT_SCORE_SIGMOID 1
struct KtRouter {
  int score;                          /* KT_SCORE_* */
  float scale;                        /* sigmoid: the weights' factor */
  const float* bias;                  /* sigmoid: [E] */
};

/* the k largest of E <= 1024 logits by one wave, the logits in registers (lane l holds e = l + 64 i, loaded together,
   clamped). Each logit becomes a 32-bit key whose unsigned order is the logits' order: the float's bits made
   order-preserving (-0 taken as +0; NaN 1, below every number; chosen and absent entries 0, below NaN, so the picks
   stay distinct while a token has k entries). A round takes the wave max of the
   keys (lane max, then an xor butterfly of unsigned maxima on the VALU exchanges, no branches) and the lowest index
   holding it (one ballot per register slot: slot i holds indices 64 i .. 64 i + 63), so ties go to the lower index;
   that entry's key is cleared. Pick j lands in lane j, which writes ids[j] and the weight exp(l_j - l_max) / sum of
   the chosen (sigmoid: s_j / sum of the chosen s * scale; either sum in j order, as a sequential loop over the
   picks). With the sigmoid scoring the key is that of s_e + bias[e]. Returns lane j's pick (lanes >= k: the last
   one). */
__device__ __forceinline__ unsigned kt_key(float x){
  unsigned u = __float_as_uint(x);
  u = u == 0x80000000u ? 0u : u;                                  /* -0 = +0 */
  const unsigned k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return x != x ? 1u : k;                                         /* NaN: never chosen before a number */
}
__device__ __forceinline__ float kt_key_val(unsigned k){
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}
template <int NI>   /* logits a lane: E <= 64 NI */
__device__ __forceinline__ int kt_topk_wave_n(const float* __restrict__ l, int E, int k, const KtRouter rt,
                                              int* __restrict__ ids, float* __restrict__ gw, int lane){
  unsigned key[NI];
  float sc[NI];                                                   /* sigmoid: the scores */
  const bool sig = rt.score == KT_SCORE_SIGMOID;                  /* uniform */
#pragma unroll
  for(int i = 0; i < NI; ++i){
    const int e = lane + 64 * i, ec = e < E ? e : E - 1;
    float x = l[ec];
    if(sig){
      sc[i] = 1.0f / (1.0f + expf(-x));
      x = sc[i] + rt.bias[ec];
    }
    key[i] = e < E ? kt_key(x) : 0u;
  }
  int mine = 0;
  float myv = 0.0f;
  for(int j = 0; j < k; ++j){                                      /* uniform */
    unsigned m = key[0];
#pragma unroll
    for(int i = 1; i < NI; ++i) m = key[i] > m ? key[i] : m;
    m = max(m, (unsigned)kf_xor<1>((int)m));
    m = max(m, (unsigned)kf_xor<2>((int)m));
    m = max(m, (unsigned)kf_xor<4>((int)m));
    m = max(m, (unsigned)kf_xor<8>((int)m));
    m = max(m, (unsigned)kf_xor<16>((int)m));
    m = max(m, (unsigned)kf_xor<32>((int)m));
    m = __builtin_amdgcn_readfirstlane(m);
    /* the lowest index holding m: the first slot with a holder, its lowest lane */
    int idx = 0x7FFFFFFF;
#pragma unroll
    for(int i = NI - 1; i >= 0; --i){
      const unsigned long long b = __ballot(key[i] == m);
      idx = b ? 64 * i + (int)__builtin_ctzll(b) : idx;
    }
    float v = kt_key_val(m);
    if(sig){                                                       /* the chosen expert's score, from its lane */
      float s = sc[0];
#pragma unroll
      for(int i = 1; i < NI; ++i) s = (idx >> 6) == i ? sc[i] : s;
      v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), idx & 63));
    }
#pragma unroll
    for(int i = 0; i < NI; ++i) key[i] = (lane + 64 * i == idx) ? 0u : key[i];
    mine = lane == j ? idx : mine;
    myv = lane == j ? v : myv;
  }
  float p = myv;
  if(!sig){
    const float lmax = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(myv)));
    p = expf(myv - lmax);
  }
  float sum = 0.0f;
  for(int j = 0; j < k; ++j) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), j));
  if(lane < k){ ids[lane] = mine; gw[lane] = sig ? p / sum * rt.scale : p / sum; }
  return mine;
}
/* the scan length by E (uniform): a lane scans only the logits it holds */
__device__ __forceinline__ int kt_topk_wave(const float* __restrict__ l, int E, int k, const KtRouter rt,
                                            int* __restrict__ ids, float* __restrict__ gw, int lane){
  if(E <= 128) return kt_topk_wave_n<2>(l, E, k, rt, ids, gw, lane);
  if(E <= 256) return kt_topk_wave_n<4>(l, E, k, rt, ids, gw, lane);
  return kt_topk_wave_n<16>(l, E, k, rt, ids, gw, lane);
}
