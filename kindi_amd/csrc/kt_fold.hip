/* kt_fold.hip - the producers of a product's input, fused with its int8 quantization (k_rmsfold_qT, k_fold_fwht_qT,
   k_smfold_qT tcf.cu:370-426; their numbers are those of k_rmsfold kindi.cu:350-394 and ff_* tcf.cu:218-312).

   One block of 512 threads per token row and chunk of CW = 512 NM columns (whole HB blocks, grid.x of them; NM <=
   16): thread j holds columns c0 + j + 512 k in v[k], and every output of the chunk is made in the block. Few
   tokens: one HB block a chunk, so a row's work is spread over C / HB blocks (the reference's grid); many tokens: the
   widest chunk (rmsfold: the whole row), so the row is read once. rmsfold's blocks each read the whole row (NF = C /
   512 registers) for the norm, in the reference's order, as every block of the reference does:
     MODE 0 (rmsfold): xf = x + (r_0 + ... + r_{n-1}) (parts in order), s = 1 / sqrt((float)(S / C) + 1e-6) with S
                       the double sum of squares, xn = (xf s) w, v = sg xn;
     MODE 1 (fold):    v = sg x;
     MODE 2 (smfold):  v = sg[e] (SiLU(a) b) at the permuted source column of e;
   then the unnormalised Walsh-Hadamard transform of each HB-column block, the 1/sqrt(HB) scale (xo), and the int8 row
   per 128-column group with k_tc_q8's numbers (natural column order, XS/XA [M][C/128] as kt_quant_q8 writes them).

   Bit-exact with the reference:
   - S is summed in the reference's order: thread j over k in order; each 32-lane half of a wave by the xor butterfly
     16, 8, 4, 2, 1 (the reference's warp); the 16 half-wave sums by the same butterfly (its warp 0 with lanes 16 ..
     31 zero), which every thread evaluates from LDS. sqrt and the division go through double, which rounds to the
     correctly rounded fp32 results the reference's IEEE sqrtf and division give.
   - The transform's butterflies are the reference's pairs in the reference's stage order: stages 1 .. 32 between
     lanes of a wave; stages 64, 128, 256 (between the 8 waves) as one LDS exchange after which each thread runs the
     8-point transform of its column's 8 values (the same additions in the same order) and keeps its own output;
     stages 512 and up between the registers of one HB block. */
#include "kt_gemv.h"
#include "kt_fold.h"
#include "kt_launch.h"

/* one butterfly stage between lanes l and l ^ X: the lower lane keeps a + b, the upper a - b, as (-b) + a: negation
   is exact and the sum is the same rounded value. neg = the sign bit on lanes with bit X set. */
template <int X> __device__ __forceinline__ float kf_bfly(float v, unsigned neg){
  return __int_as_float(__float_as_int(v) ^ neg) + kf_xorf<X>(v);
}
__device__ __forceinline__ float kf_wave_max(float m){   /* every lane: the wave's maximum */
  m = fmaxf(m, kf_xorf<1>(m)); m = fmaxf(m, kf_xorf<2>(m)); m = fmaxf(m, kf_xorf<4>(m));
  m = fmaxf(m, kf_xorf<8>(m)); m = fmaxf(m, kf_xorf<16>(m)); return fmaxf(m, kf_xorf<32>(m));
}
__device__ __forceinline__ int kf_wave_sum(int v){
  v += kf_xor<1>(v); v += kf_xor<2>(v); v += kf_xor<4>(v); v += kf_xor<8>(v); v += kf_xor<16>(v);
  return v + kf_xor<32>(v);
}

template <int NM>
__device__ __forceinline__ void kf_fwht(float* v, float* sm, int j, int HB){
  const int l = j & 63;
#define KF_STAGE(X) { const unsigned ng = (l & X) ? 0x80000000u : 0u; \
    _Pragma("unroll") for(int k = 0; k < NM; ++k) v[k] = kf_bfly<X>(v[k], ng); }
  KF_STAGE(1) KF_STAGE(2) KF_STAGE(4) KF_STAGE(8) KF_STAGE(16) KF_STAGE(32)
#undef KF_STAGE
#pragma unroll
  for(int k = 0; k < NM; ++k) sm[k * 512 + j] = v[k];
  __syncthreads();
  /* stages 64, 128, 256 for this thread's column only: with A_t = the column's value in wave w ^ t,
     s1_t = stage 64 at wave w ^ t (t even), s2_t = stage 128 at w ^ t (t = 0, 4), then stage 256 at w; each is the
     reference's a + b or a - b of the same pair (the lower wave of a pair adds) */
  const int w = __builtin_amdgcn_readfirstlane(j >> 6);
#pragma unroll
  for(int k = 0; k < NM; ++k){
    float A[8];
#pragma unroll
    for(int t = 0; t < 8; ++t) A[t] = sm[k * 512 + l + 64 * (w ^ t)];
    float s1[8], s2[8];
#pragma unroll
    for(int t = 0; t < 8; t += 2) s1[t] = (w & 1) ? (A[t ^ 1] - A[t]) : (A[t] + A[t ^ 1]);
#pragma unroll
    for(int t = 0; t < 8; t += 4) s2[t] = (w & 2) ? (s1[t ^ 2] - s1[t]) : (s1[t] + s1[t ^ 2]);
    v[k] = (w & 4) ? (s2[4] - s2[0]) : (s2[0] + s2[4]);
  }
  const int hbe = HB >> 9;                                     /* registers a Hadamard block */
#pragma unroll
  for(int h = 1; h < 16; h <<= 1){
    if(h < hbe){
#pragma unroll
      for(int k = 0; k < NM; ++k)
        if(!(k & h) && k + h < NM){ const float a = v[k], b = v[k + h]; v[k] = a + b; v[k + h] = a - b; }
    }
  }
}

template <int MODE, int NM, int NF>
__global__ void __launch_bounds__(512) k_fold_q8(const KtFoldArgs a){
  __shared__ float sm[NM * 512];
  __shared__ double red[16];
  __shared__ float qm[NM * 8];
  __shared__ int qs[NM * 8], qs2[NM * 8];
  const int j = threadIdx.x, n = blockIdx.y, lane = j & 63, w = j >> 6, C = NM * 512, c0 = blockIdx.x * C;
  float v[NM];
  if(MODE == 0){
    const float* x = a.x + (long long)n * a.ldx;
    constexpr int CF = NF * 512;                                   /* the row */
    float xf[NF], wv[NM], sv[NM];
#pragma unroll
    for(int m = 0; m < NF; ++m) xf[m] = x[j + 512 * m];
#pragma unroll
    for(int k = 0; k < NM; ++k){ wv[k] = a.w[c0 + j + 512 * k]; sv[k] = a.sg[c0 + j + 512 * k]; }
    if(a.nparts > 0){
      const float* r = a.r + (long long)n * a.ldr;
      float rv[NF];
#pragma unroll
      for(int m = 0; m < NF; ++m) rv[m] = r[j + 512 * m];
      for(int p = 1; p < a.nparts; ++p){
#pragma unroll
        for(int m = 0; m < NF; ++m) rv[m] += r[(long long)p * CF + j + 512 * m];
      }
#pragma unroll
      for(int m = 0; m < NF; ++m) xf[m] = xf[m] + rv[m];
    }
    double acc = 0.0;
#pragma unroll
    for(int m = 0; m < NF; ++m){ const double d = (double)xf[m]; acc += d * d; }
    acc += kf_xord<16>(acc);
    acc += kf_xord<8>(acc);
    acc += kf_xord<4>(acc);
    acc += kf_xord<2>(acc);
    acc += kf_xord<1>(acc);
    if((j & 31) == 0) red[j >> 5] = acc;
    __syncthreads();
    double t[8];
#pragma unroll
    for(int i = 0; i < 8; ++i) t[i] = red[i] + red[i + 8];         /* offset 8 (offset 16 added zeros) */
#pragma unroll
    for(int i = 0; i < 4; ++i) t[i] = t[i] + t[i + 4];
    t[0] = t[0] + t[2];
    t[1] = t[1] + t[3];
    const double S = t[0] + t[1];
    const float ms = (float)(S / (double)CF) + 1e-6f;
    const float q = (float)sqrt((double)ms);
    const float s = (float)(1.0 / (double)q);
    float* xw = a.xw ? a.xw + (long long)n * a.ldxw : nullptr;
    float* xn = a.xn ? a.xn + (long long)n * a.ldxn : nullptr;
    const int b0 = blockIdx.x * NM;                                /* the chunk's first register of the row */
#pragma unroll
    for(int k = 0; k < NM; ++k){
      const int e = c0 + j + 512 * k;
      float f = xf[k];
#pragma unroll
      for(int m = 0; m < NF; ++m) if(m != k && m == b0 + k) f = xf[m];
      const float nv = (f * s) * wv[k];
      if(xw && a.nparts > 0) xw[e] = f;
      if(xn) xn[e] = nv;
      v[k] = sv[k] * nv;
    }
  } else if(MODE == 1){
    const float* x = a.x + (long long)n * a.ldx;
#pragma unroll
    for(int k = 0; k < NM; ++k) v[k] = a.sg[c0 + j + 512 * k] * x[c0 + j + 512 * k];
  } else {
    const float* pa = a.x + (long long)n * a.ldx;
    const float* pb = a.r + (long long)n * a.ldr;
#pragma unroll
    for(int k = 0; k < NM; ++k){
      const int e = c0 + j + 512 * k;
      int src = e;
      if(a.rep > 1){
        const int h = e % a.hd, g = e / a.hd, rp = g % a.rep, kk = g / a.rep;
        src = h + a.hd * (kk + a.nk * rp);
      }
      const float xa = pa[src];
      const float m = (xa / (1.0f + expf(-xa))) * pb[src];
      v[k] = a.sg[e] * m;
    }
  }
  kf_fwht<NM>(v, sm, j, a.HB);
  const float sc = a.HB == 512 ? 0.044194173824159220878f : (a.HB == 1024 ? 0.03125f : 0.015625f);
  float* xo = a.xo ? a.xo + (long long)n * a.ldxo : nullptr;
#pragma unroll
  for(int k = 0; k < NM; ++k){
    v[k] = v[k] * sc;
    if(xo) xo[c0 + j + 512 * k] = v[k];
  }
  /* group 4 k + w / 2 = waves 2i, 2i + 1 of register k */
#pragma unroll
  for(int k = 0; k < NM; ++k){
    const float m = kf_wave_max(fabsf(v[k]));
    if(lane == 0) qm[k * 8 + w] = m;
  }
  __syncthreads();
  /* hp: rows 2n (the int8 row) and 2n + 1 (the residual r = v - q (amax / 127), one fma as the reference's compiler
     contracts it, at the fixed scale amax / 32258: q2 = clamp(rne(r (32258 / amax)), -127, 127); ff_q8 tcf.cu:150-205) */
  const long long n0 = a.hp ? 2 * n : n;
  int8_t* Q = a.Q + n0 * a.ldq;
  const int NG = a.C >> 7;
#pragma unroll
  for(int k = 0; k < NM; ++k){
    const float amax = fmaxf(qm[k * 8 + (w & ~1)], qm[k * 8 + (w | 1)]);
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    const int qi = __float2int_rn(v[k] * id);
    Q[c0 + j + 512 * k] = (int8_t)qi;
    const int sum = kf_wave_sum(qi);
    if(lane == 0) qs[k * 8 + w] = sum;
    if(a.hp){                                                    /* block-uniform */
      const float r = fmaf(-(float)qi, amax / 127.0f, v[k]);
      const int q2 = max(-127, min(127, __float2int_rn(r * (amax != 0.0f ? 32258.0f / amax : 0.0f))));
      Q[a.ldq + c0 + j + 512 * k] = (int8_t)q2;
      const int sum2 = kf_wave_sum(q2);
      if(lane == 0) qs2[k * 8 + w] = sum2;
    }
  }
  __syncthreads();
  if(lane == 0 && !(w & 1)){
#pragma unroll
    for(int k = 0; k < NM; ++k){
      const int g = (c0 >> 7) + 4 * k + (w >> 1);
      const float amax = fmaxf(qm[k * 8 + w], qm[k * 8 + w + 1]);
      a.XS[n0 * NG + g] = amax / 127.0f;
      a.XA[n0 * NG + g] = qs[k * 8 + w] + qs[k * 8 + w + 1];
      if(a.hp){
        a.XS[(n0 + 1) * NG + g] = amax / 32258.0f;
        a.XA[(n0 + 1) * NG + g] = qs2[k * 8 + w] + qs2[k * 8 + w + 1];
      }
    }
  }
}

/* rmsfold: (chunk, row) = (HB block, row) and (row, row); fold / smfold: chunks of 1 .. 16 registers */
template __global__ void k_fold_q8<0, 1, 1>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 1, 2>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 1, 3>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 1, 4>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 1, 5>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 1, 6>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 1, 7>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 1, 8>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 1, 9>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 1, 10>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 1, 11>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 1, 12>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 1, 13>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 1, 14>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 1, 15>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 1, 16>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 2, 2>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 2, 4>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 2, 6>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 2, 8>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 2, 10>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 2, 12>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 2, 14>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 2, 16>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 3, 3>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 4, 4>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 5, 5>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 6, 6>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 7, 7>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 8, 8>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 8, 16>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 9, 9>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 10, 10>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 11, 11>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 12, 12>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 13, 13>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 14, 14>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 15, 15>(const KtFoldArgs);
template __global__ void k_fold_q8<0, 16, 16>(const KtFoldArgs);
template __global__ void k_fold_q8<1, 1, 1>(const KtFoldArgs);
template __global__ void k_fold_q8<1, 2, 2>(const KtFoldArgs);
template __global__ void k_fold_q8<1, 3, 3>(const KtFoldArgs);
template __global__ void k_fold_q8<1, 4, 4>(const KtFoldArgs);
template __global__ void k_fold_q8<1, 5, 5>(const KtFoldArgs);
template __global__ void k_fold_q8<1, 6, 6>(const KtFoldArgs);
template __global__ void k_fold_q8<1, 7, 7>(const KtFoldArgs);
template __global__ void k_fold_q8<1, 8, 8>(const KtFoldArgs);
template __global__ void k_fold_q8<1, 9, 9>(const KtFoldArgs);
template __global__ void k_fold_q8<1, 10, 10>(const KtFoldArgs);
template __global__ void k_fold_q8<1, 11, 11>(const KtFoldArgs);
template __global__ void k_fold_q8<1, 12, 12>(const KtFoldArgs);
template __global__ void k_fold_q8<1, 13, 13>(const KtFoldArgs);
template __global__ void k_fold_q8<1, 14, 14>(const KtFoldArgs);
template __global__ void k_fold_q8<1, 15, 15>(const KtFoldArgs);
template __global__ void k_fold_q8<1, 16, 16>(const KtFoldArgs);
template __global__ void k_fold_q8<2, 1, 1>(const KtFoldArgs);
template __global__ void k_fold_q8<2, 2, 2>(const KtFoldArgs);
template __global__ void k_fold_q8<2, 3, 3>(const KtFoldArgs);
template __global__ void k_fold_q8<2, 4, 4>(const KtFoldArgs);
template __global__ void k_fold_q8<2, 5, 5>(const KtFoldArgs);
template __global__ void k_fold_q8<2, 6, 6>(const KtFoldArgs);
template __global__ void k_fold_q8<2, 7, 7>(const KtFoldArgs);
template __global__ void k_fold_q8<2, 8, 8>(const KtFoldArgs);
template __global__ void k_fold_q8<2, 9, 9>(const KtFoldArgs);
template __global__ void k_fold_q8<2, 10, 10>(const KtFoldArgs);
template __global__ void k_fold_q8<2, 11, 11>(const KtFoldArgs);
template __global__ void k_fold_q8<2, 12, 12>(const KtFoldArgs);
template __global__ void k_fold_q8<2, 13, 13>(const KtFoldArgs);
template __global__ void k_fold_q8<2, 14, 14>(const KtFoldArgs);
template __global__ void k_fold_q8<2, 15, 15>(const KtFoldArgs);
template __global__ void k_fold_q8<2, 16, 16>(const KtFoldArgs);

#define KF_KEY(MODE, NM, NF) ((MODE) * 1024 + (NM) * 32 + (NF))
#define KF_FEW 32                     /* up to this many tokens, one HB block a chunk */

/* host launcher (kt_api.hip validates the arguments) */
static bool kf_overlap(const float* p, int ldp, const float* q, int ldq, int M, int C){
  if(!p || !q) return false;
  const uintptr_t p0 = (uintptr_t)p, p1 = p0 + ((size_t)(M - 1) * ldp + C) * 4;
  const uintptr_t q0 = (uintptr_t)q, q1 = q0 + ((size_t)(M - 1) * ldq + C) * 4;
  return p0 < q1 && q0 < p1;
}

hipError_t kt_fold_launch(int mode, const KtFoldArgs& a, int M, hipStream_t s){
  int cw = a.HB;
  /* rmsfold over chunks of a row: every chunk's block reads the whole row (x and the parts, for the norm) while it
     writes its own chunk of xw / xn / xo. When one of those outputs overlaps x or the parts, one block takes the row
     (each thread writes only the columns it has read), so no block can overwrite what another has still to read. */
  const int np = a.nparts > 0 ? a.nparts : 0;
  const bool alias = mode == 0 && (kf_overlap(a.xw, a.ldxw, a.x, a.ldx, M, a.C) || kf_overlap(a.xn, a.ldxn, a.x, a.ldx, M, a.C)
      || kf_overlap(a.xo, a.ldxo, a.x, a.ldx, M, a.C) || (np && (kf_overlap(a.xw, a.ldxw, a.r, a.ldr, M, np * a.C)
      || kf_overlap(a.xn, a.ldxn, a.r, a.ldr, M, np * a.C) || kf_overlap(a.xo, a.ldxo, a.r, a.ldr, M, np * a.C))));
  if(M > KF_FEW || alias){
    if(mode == 0) cw = a.C;
    else for(cw = (8192 / a.HB) * a.HB; cw > a.HB && a.C % cw; cw -= a.HB) {}
  }
  const int nm = cw >> 9, nf = mode == 0 ? a.C >> 9 : nm;
  void (*k)(const KtFoldArgs) = nullptr;
  switch(KF_KEY(mode, nm, nf)){
    case KF_KEY(0, 1, 1): k = k_fold_q8<0, 1, 1>; break;
    case KF_KEY(0, 1, 2): k = k_fold_q8<0, 1, 2>; break;
    case KF_KEY(0, 1, 3): k = k_fold_q8<0, 1, 3>; break;
    case KF_KEY(0, 1, 4): k = k_fold_q8<0, 1, 4>; break;
    case KF_KEY(0, 1, 5): k = k_fold_q8<0, 1, 5>; break;
    case KF_KEY(0, 1, 6): k = k_fold_q8<0, 1, 6>; break;
    case KF_KEY(0, 1, 7): k = k_fold_q8<0, 1, 7>; break;
    case KF_KEY(0, 1, 8): k = k_fold_q8<0, 1, 8>; break;
    case KF_KEY(0, 1, 9): k = k_fold_q8<0, 1, 9>; break;
    case KF_KEY(0, 1, 10): k = k_fold_q8<0, 1, 10>; break;
    case KF_KEY(0, 1, 11): k = k_fold_q8<0, 1, 11>; break;
    case KF_KEY(0, 1, 12): k = k_fold_q8<0, 1, 12>; break;
    case KF_KEY(0, 1, 13): k = k_fold_q8<0, 1, 13>; break;
    case KF_KEY(0, 1, 14): k = k_fold_q8<0, 1, 14>; break;
    case KF_KEY(0, 1, 15): k = k_fold_q8<0, 1, 15>; break;
    case KF_KEY(0, 1, 16): k = k_fold_q8<0, 1, 16>; break;
    case KF_KEY(0, 2, 2): k = k_fold_q8<0, 2, 2>; break;
    case KF_KEY(0, 2, 4): k = k_fold_q8<0, 2, 4>; break;
    case KF_KEY(0, 2, 6): k = k_fold_q8<0, 2, 6>; break;
    case KF_KEY(0, 2, 8): k = k_fold_q8<0, 2, 8>; break;
    case KF_KEY(0, 2, 10): k = k_fold_q8<0, 2, 10>; break;
    case KF_KEY(0, 2, 12): k = k_fold_q8<0, 2, 12>; break;
    case KF_KEY(0, 2, 14): k = k_fold_q8<0, 2, 14>; break;
    case KF_KEY(0, 2, 16): k = k_fold_q8<0, 2, 16>; break;
    case KF_KEY(0, 3, 3): k = k_fold_q8<0, 3, 3>; break;
    case KF_KEY(0, 4, 4): k = k_fold_q8<0, 4, 4>; break;
    case KF_KEY(0, 5, 5): k = k_fold_q8<0, 5, 5>; break;
    case KF_KEY(0, 6, 6): k = k_fold_q8<0, 6, 6>; break;
    case KF_KEY(0, 7, 7): k = k_fold_q8<0, 7, 7>; break;
    case KF_KEY(0, 8, 8): k = k_fold_q8<0, 8, 8>; break;
    case KF_KEY(0, 8, 16): k = k_fold_q8<0, 8, 16>; break;
    case KF_KEY(0, 9, 9): k = k_fold_q8<0, 9, 9>; break;
    case KF_KEY(0, 10, 10): k = k_fold_q8<0, 10, 10>; break;
    case KF_KEY(0, 11, 11): k = k_fold_q8<0, 11, 11>; break;
    case KF_KEY(0, 12, 12): k = k_fold_q8<0, 12, 12>; break;
    case KF_KEY(0, 13, 13): k = k_fold_q8<0, 13, 13>; break;
    case KF_KEY(0, 14, 14): k = k_fold_q8<0, 14, 14>; break;
    case KF_KEY(0, 15, 15): k = k_fold_q8<0, 15, 15>; break;
    case KF_KEY(0, 16, 16): k = k_fold_q8<0, 16, 16>; break;
    case KF_KEY(1, 1, 1): k = k_fold_q8<1, 1, 1>; break;
    case KF_KEY(1, 2, 2): k = k_fold_q8<1, 2, 2>; break;
    case KF_KEY(1, 3, 3): k = k_fold_q8<1, 3, 3>; break;
    case KF_KEY(1, 4, 4): k = k_fold_q8<1, 4, 4>; break;
    case KF_KEY(1, 5, 5): k = k_fold_q8<1, 5, 5>; break;
    case KF_KEY(1, 6, 6): k = k_fold_q8<1, 6, 6>; break;
    case KF_KEY(1, 7, 7): k = k_fold_q8<1, 7, 7>; break;
    case KF_KEY(1, 8, 8): k = k_fold_q8<1, 8, 8>; break;
    case KF_KEY(1, 9, 9): k = k_fold_q8<1, 9, 9>; break;
    case KF_KEY(1, 10, 10): k = k_fold_q8<1, 10, 10>; break;
    case KF_KEY(1, 11, 11): k = k_fold_q8<1, 11, 11>; break;
    case KF_KEY(1, 12, 12): k = k_fold_q8<1, 12, 12>; break;
    case KF_KEY(1, 13, 13): k = k_fold_q8<1, 13, 13>; break;
    case KF_KEY(1, 14, 14): k = k_fold_q8<1, 14, 14>; break;
    case KF_KEY(1, 15, 15): k = k_fold_q8<1, 15, 15>; break;
    case KF_KEY(1, 16, 16): k = k_fold_q8<1, 16, 16>; break;
    case KF_KEY(2, 1, 1): k = k_fold_q8<2, 1, 1>; break;
    case KF_KEY(2, 2, 2): k = k_fold_q8<2, 2, 2>; break;
    case KF_KEY(2, 3, 3): k = k_fold_q8<2, 3, 3>; break;
    case KF_KEY(2, 4, 4): k = k_fold_q8<2, 4, 4>; break;
    case KF_KEY(2, 5, 5): k = k_fold_q8<2, 5, 5>; break;
    case KF_KEY(2, 6, 6): k = k_fold_q8<2, 6, 6>; break;
    case KF_KEY(2, 7, 7): k = k_fold_q8<2, 7, 7>; break;
    case KF_KEY(2, 8, 8): k = k_fold_q8<2, 8, 8>; break;
    case KF_KEY(2, 9, 9): k = k_fold_q8<2, 9, 9>; break;
    case KF_KEY(2, 10, 10): k = k_fold_q8<2, 10, 10>; break;
    case KF_KEY(2, 11, 11): k = k_fold_q8<2, 11, 11>; break;
    case KF_KEY(2, 12, 12): k = k_fold_q8<2, 12, 12>; break;
    case KF_KEY(2, 13, 13): k = k_fold_q8<2, 13, 13>; break;
    case KF_KEY(2, 14, 14): k = k_fold_q8<2, 14, 14>; break;
    case KF_KEY(2, 15, 15): k = k_fold_q8<2, 15, 15>; break;
    case KF_KEY(2, 16, 16): k = k_fold_q8<2, 16, 16>; break;
    default: return hipErrorInvalidValue;
  }
  return kt_go(k, dim3(a.C / cw, M), dim3(512), 0, s, a);
}
