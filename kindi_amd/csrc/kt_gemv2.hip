/* kt_gemv2.hip - the one-token ternary decode product with two row groups a block (k_gemv_pair), for launches whose
   one-row-group grid (k_gemv_flat1) would not fit the GPU's wave slots at once (the 27B-class gate/up pair: 4352 row
   groups x 3 K slices = 13056 waves against 8192 slots, so a second round of blocks would issue its loads only after
   the first round has finished).

   A block takes row groups 2 b and 2 b + 1 of the launch's matrices (every matrix has an even number of row groups); wave ks takes K slice ks of both, issues the code
   and scale loads of both and the activation row of the slice at once (one memory round trip), stages the
   activations in LDS once for both, and computes each row group exactly as k_gemv_flat1 does: lane c chains
   fmaf((float)(v - XA), XS d, .) over its units of the slice, the xor butterfly adds the 8 lanes of a row, and the
   slice sums are added in slice order. So every row has the same bits as on k_gemv_flat1 (the tree depends on C
   only). */
#include "kt_gemv.h"

/* kt_unit_lds for two row groups' code words against one unit's staged activations: each half's four activation
   chunks are read once and feed both (integer sums: the same values as two kt_unit_lds calls), one half at a time so
   that only four chunks are live */
__device__ __forceinline__ void kt_unit2_lds(const uint4 a0c, const uint4 a1c, const uint4 b0c, const uint4 b1c,
                                             const uint8_t* xrow, int (&v)[2]){
  const uint4* q = (const uint4*)xrow;
  int s0[3] = {0, 0, 0}, s1[3] = {0, 0, 0};
#pragma unroll
  for(int h = 0; h < 2; ++h){
    const uint4 ca = h ? a1c : a0c, cb = h ? b1c : b0c;
    const uint32_t wa[4] = {ca.x, ca.y, ca.z, ca.w}, wb[4] = {cb.x, cb.y, cb.z, cb.w};
    uint4 x[4];
#pragma unroll
    for(int j = 0; j < 4; ++j) x[j] = q[4 * h + j];
#pragma unroll
    for(int j = 0; j < 4; ++j){
      s0[0] = kt_dot4((int)(wa[j] & 0x03030303u), (int)x[j].x, s0[0]);
      s0[1] = kt_dot4((int)(wa[j] & 0x0C0C0C0Cu), (int)x[j].y, s0[1]);
      s0[2] = kt_dot4((int)(wa[j] & 0x30303030u), (int)x[j].z, s0[2]);
      s0[0] = kt_dot4((int)((wa[j] >> 6) & 0x03030303u), (int)x[j].w, s0[0]);
      s1[0] = kt_dot4((int)(wb[j] & 0x03030303u), (int)x[j].x, s1[0]);
      s1[1] = kt_dot4((int)(wb[j] & 0x0C0C0C0Cu), (int)x[j].y, s1[1]);
      s1[2] = kt_dot4((int)(wb[j] & 0x30303030u), (int)x[j].z, s1[2]);
      s1[0] = kt_dot4((int)((wb[j] >> 6) & 0x03030303u), (int)x[j].w, s1[0]);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  v[0] = s0[0] + (s0[1] >> 2) + (s0[2] >> 4);
  v[1] = s1[0] + (s1[1] >> 2) + (s1[2] >> 4);
}

/* 7 waves a SIMD (72 VGPRs): 7168 wave slots, enough for the pair grid of the 27B gate/up launch (6528 waves) */
template <bool DBG>
__global__ void __launch_bounds__(64 * KT_KSMAX) __attribute__((amdgpu_waves_per_eu(7)))
k_gemv_pair(const KtGemvArgs a, const int8_t* __restrict__ xq, const float* __restrict__ xs,
            const int* __restrict__ xa, int32_t* __restrict__ dbg, int KS){
  extern __shared__ __attribute__((aligned(16))) uint8_t kt_lds[];
  using F = KtFlat<KT_FMT_TERN, 1>;
  constexpr int UW = F::UW, UP = F::UP, SL = KT_SL;
  const int NU = a.NU, S = kt_steps(NU);
  const int lane = threadIdx.x & 63, ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), r = lane & 7, c = lane >> 3;
  const int s_lo = ks * S / KS, ns = (ks + 1) * S / KS - s_lo;      /* 1 or 2 steps (the launcher checks) */
  uint8_t* xw = kt_lds + (size_t)ks * F::XW;                         /* [SL][8][UP] */
  float* red = (float*)(kt_lds + (size_t)KS * F::XW);                /* [KS][2][8] */

  /* both row groups are in one matrix (every matrix of the launch has an even number of row groups: the launcher
     checks), so the second one's loads are the first one's offsets from bases one row group further */
  const int g = 2 * blockIdx.x;
  int mi = 0;
  if(a.nmat > 1 && g >= a.mat[1].rg0) mi = 1;
  if(a.nmat > 2 && g >= a.mat[2].rg0) mi = 2;
  const KtMat& m = a.mat[mi];
  const int rg0 = g - m.rg0, R = m.R;
  const uint4* wb0 = (const uint4*)m.codes;
  const uint16_t* sb0 = m.scales;
  const uint4* wb1 = wb0 + (long long)NU * 16;
  const uint16_t* sb1 = sb0 + (long long)NU * 8;
  float* yo = m.y;
  KtStep w[2][SL];
  unsigned o0[SL], o1[SL], os[SL];
#pragma unroll
  for(int j = 0; j < SL; ++j){
    const int s = s_lo + j, u = s * KT_KL + c;
    const bool ok = j < ns && u < NU;
    o0[j] = ok ? (unsigned)kt_widx(NU, rg0, s, 0, c, r) : 0u;
    o1[j] = ok ? (unsigned)kt_widx(NU, rg0, s, 1, c, r) : 0u;
    os[j] = ok ? (unsigned)kt_sidx(NU, rg0, u, r) : 0u;
  }
#pragma unroll
  for(int j = 0; j < SL; ++j){
    w[0][j].c0 = kt_ldnt(wb0 + o0[j]);
    w[0][j].c1 = kt_ldnt(wb0 + o1[j]);
    w[0][j].hs = sb0[os[j]];
    w[1][j].c0 = kt_ldnt(wb1 + o0[j]);
    w[1][j].c1 = kt_ldnt(wb1 + o1[j]);
    w[1][j].hs = sb1[os[j]];
  }
  /* the slice's activations (token 0): each lane's 16 bytes of a step's row, its unit's scale and sum */
  uint32_t sa[2][SL];
  uint4 stg[SL];
  const int o = lane * 16;
#pragma unroll
  for(int j = 0; j < SL; ++j){
    const int s = s_lo + (j < ns ? j : 0), u = s * KT_KL + c, uu = (j < ns && u < NU) ? u : 0;
    const int nc = NU - s * KT_KL < KT_KL ? NU - s * KT_KL : KT_KL;
    sa[0][j] = __float_as_uint(xs[uu]);
    sa[1][j] = (uint32_t)xa[uu];
    const int oc = o < nc * UW ? o : 0;
    stg[j] = *(const uint4*)(xq + (long long)s * KT_KL * UW + oc);
  }
  kt_pin<SL>(&stg[0], &sa[0][0]);
#pragma unroll
  for(int j = 0; j < SL; ++j) *(uint4*)(xw + j * KT_KL * UP + (o / UW) * UP + o % UW) = stg[j];
  kt_wave_sync();
  float acc[2] = {0.0f, 0.0f};
#pragma unroll
  for(int j = 0; j < SL; ++j){
    const int u = (s_lo + j) * KT_KL + c;
    if(j < ns){                                                      /* wave-uniform */
      const bool uok = u < NU;
      int vv[2];
      kt_unit2_lds(w[0][j].c0, w[0][j].c1, w[1][j].c0, w[1][j].c1, xw + (j * KT_KL + (uok ? c : 0)) * UP, vv);
#pragma unroll
      for(int q = 0; q < 2; ++q){
        const float d = uok ? kt_h2f(w[q][j].hs) : 0.0f;
        const int v = uok ? vv[q] - (int)sa[1][j] : 0;
        acc[q] = fmaf((float)v, __uint_as_float(sa[0][j]) * d, acc[q]);
        const int row = (rg0 + q) * KT_RG + r;
        if(DBG && uok && row < R) dbg[(long long)row * NU + u] = v;
      }
    }
  }
#pragma unroll
  for(int q = 0; q < 2; ++q){
    const float y = kt_row_sum(acc[q]);
    if(c == q) red[(ks * 2 + q) * 8 + r] = y;
  }
  __syncthreads();
  /* lanes 8 q + r of wave 0: row r of row group q, the slice sums in slice order */
  if(ks == 0 && c < 2){
    const int q = c, row = (rg0 + q) * KT_RG + r;
    float v = red[q * 8 + r];
    for(int k = 1; k < KS; ++k) v += red[(k * 2 + q) * 8 + r];
    if(row < R) yo[row] = v;
  }
}

template __global__ void k_gemv_pair<false>(const KtGemvArgs, const int8_t*, const float*, const int*, int32_t*, int);
template __global__ void k_gemv_pair<true>(const KtGemvArgs, const int8_t*, const float*, const int*, int32_t*, int);

/* ------------------------------------------------------------------ one step a wave
   k_gemv_step: the one-token ternary product for rows of up to 8 steps (C <= 8192) with the work of a K slice split
   over its steps: wave j of a block takes step j (8 units) of RG row groups (RG = 2: the pair kernel's grid, for
   launches too large for the wave slots). It loads its step's codes, scales and activation row (one memory round
   trip, half of a two-step slice's bytes, so the wave finishes sooner), computes each lane's exact unit value as
   k_gemv_flat1 does, and writes (float)(v - XA) and XS d (the same product k_gemv_flat1 forms) to LDS. After one
   block barrier wave 0 runs, for every K slice (kt_decode_kslices, unchanged), each lane's chain over the slice's
   steps in order, fmaf(f, m, 0) then fmaf(f, m, acc), the xor butterfly and the slice sums left to right: the same
   operations in the same order as k_gemv_flat1, so the same bits. */
template <int RG, bool DBG>
__global__ void __launch_bounds__(64 * 8) __attribute__((amdgpu_waves_per_eu(8)))
k_gemv_step(const KtGemvArgs a, const int8_t* __restrict__ xq, const float* __restrict__ xs,
            const int* __restrict__ xa, int32_t* __restrict__ dbg, int KS){
  extern __shared__ __attribute__((aligned(16))) uint8_t kt_lds[];
  using F = KtFlat<KT_FMT_TERN, 1>;
  constexpr int UW = F::UW, UP = F::UP;
  const int NU = a.NU, S = kt_steps(NU);
  const int lane = threadIdx.x & 63, j = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), r = lane & 7, c = lane >> 3;
  uint8_t* xw = kt_lds + (size_t)j * KT_KL * UP;                    /* this wave's step: [8 units][UP] */
  float* fv = (float*)(kt_lds + (size_t)S * KT_KL * UP);            /* [RG][S][64]: (float)(v - XA) */
  float* mv = fv + RG * S * 64;                                     /* [RG][S][64]: XS d */

  /* the block's row groups are in one matrix (RG = 2: every matrix has an even number of row groups, the launcher
     checks) */
  const int g = RG * blockIdx.x;
  int mi = 0;
  if(a.nmat > 1 && g >= a.mat[1].rg0) mi = 1;
  if(a.nmat > 2 && g >= a.mat[2].rg0) mi = 2;
  const KtMat& m = a.mat[mi];
  const int rg0 = g - m.rg0, R = m.R;
  const uint4* wb = (const uint4*)m.codes;
  const uint16_t* sb = m.scales;
  const int u = j * KT_KL + c;
  const bool uok = u < NU;
  const unsigned o0 = uok ? (unsigned)kt_widx(NU, rg0, j, 0, c, r) : 0u;
  const unsigned o1 = uok ? (unsigned)kt_widx(NU, rg0, j, 1, c, r) : 0u;
  const unsigned os = uok ? (unsigned)kt_sidx(NU, rg0, uok ? u : 0, r) : 0u;
  /* the step's activation row (token 0) first: each lane's 16 bytes, its unit's scale and sum; loads retire in order,
     so the staging below waits for these alone while the weights are still in flight, and the first halves of the
     units (c0 of every row group, loaded before the c1 halves) can start before the last weight bytes land
     (measured on MI355X, 27B-class step at one token against the weights first: 1.824 -> 1.803 ms) */
  const int nc = NU - j * KT_KL < KT_KL ? NU - j * KT_KL : KT_KL;
  const int o = lane * 16, oc = o < nc * UW ? o : 0;
  uint4 stg = *(const uint4*)(xq + (long long)j * KT_KL * UW + oc);
  uint32_t sa[2] = {__float_as_uint(xs[uok ? u : 0]), (uint32_t)xa[uok ? u : 0]};
  KtStep w[RG];
#pragma unroll
  for(int q = 0; q < RG; ++q) w[q].c0 = kt_ldnt(wb + (long long)q * NU * 16 + o0);
#pragma unroll
  for(int q = 0; q < RG; ++q) w[q].c1 = kt_ldnt(wb + (long long)q * NU * 16 + o1);
#pragma unroll
  for(int q = 0; q < RG; ++q) w[q].hs = sb[(long long)q * NU * 8 + os];
  __builtin_amdgcn_sched_barrier(0);
  kt_pin<1>(&stg, sa);
  *(uint4*)(xw + (o / UW) * UP + o % UW) = stg;
  kt_wave_sync();
  int vv[2];
  if(RG == 2) kt_unit2_lds(w[0].c0, w[0].c1, w[1].c0, w[1].c1, xw + (uok ? c : 0) * UP, vv);
  else vv[0] = kt_unit_lds<KT_FMT_TERN>(w[0].c0, w[0].c1, xw + (uok ? c : 0) * UP);
#pragma unroll
  for(int q = 0; q < RG; ++q){
    const float d = uok ? kt_h2f(w[q].hs) : 0.0f;
    const int v = uok ? vv[q] - (int)sa[1] : 0;
    fv[(q * S + j) * 64 + lane] = (float)v;
    mv[(q * S + j) * 64 + lane] = __uint_as_float(sa[0]) * d;
    const int row = (rg0 + q) * KT_RG + r;
    if(DBG && uok && row < R) dbg[(long long)row * NU + u] = v;
  }
  __syncthreads();
  if(j == 0){
#pragma unroll
    for(int q = 0; q < RG; ++q){
      float tot = 0.0f;
      for(int k = 0; k < KS; ++k){                                  /* uniform */
        const int s_lo = k * S / KS, ns = (k + 1) * S / KS - s_lo;
        const float* f = fv + (q * S + s_lo) * 64 + lane;
        const float* mm = mv + (q * S + s_lo) * 64 + lane;
        float acc = fmaf(f[0], mm[0], 0.0f);
        if(ns > 1) acc = fmaf(f[64], mm[64], acc);
        const float y = kt_row_sum(acc);
        tot = k == 0 ? y : tot + y;
      }
      const int row = (rg0 + q) * KT_RG + r;
      if(c == 0 && row < R) m.y[row] = tot;
    }
  }
}

template __global__ void k_gemv_step<1, false>(const KtGemvArgs, const int8_t*, const float*, const int*, int32_t*, int);
template __global__ void k_gemv_step<1, true>(const KtGemvArgs, const int8_t*, const float*, const int*, int32_t*, int);
template __global__ void k_gemv_step<2, false>(const KtGemvArgs, const int8_t*, const float*, const int*, int32_t*, int);
template __global__ void k_gemv_step<2, true>(const KtGemvArgs, const int8_t*, const float*, const int*, int32_t*, int);

/* ------------------------------------------------------------------ one step a wave, several tokens
   k_gemv_stepm: k_gemv_step for 2-5 tokens (the launcher's range below the matrix-core kernels; with the two-row form
   a token's two rows are adjacent tokens here). Wave j loads step j's codes and scales of its row group once and
   serves the tokens in chunks of MT: it stages the chunk's activation rows of its step, computes each lane's exact
   unit value per token as k_gemv_flat does, and writes (float)(v - XA) and XS d to LDS. After a block barrier wave 0
   runs, per token, every K slice's chain over its steps in order, the xor butterfly and the slice sums left to right:
   k_gemv_flat's operations in its order, so the same bits. With hp the chunk's row pairs (MT is even, so a pair never
   straddles two chunks) are added in the store. 4 waves a SIMD (76 VGPRs, no spills; 8 a SIMD spilled). */
template <int MT, bool DBG>
__global__ void __launch_bounds__(64 * 8) __attribute__((amdgpu_waves_per_eu(4)))
k_gemv_stepm(const KtGemvArgs a, const int8_t* __restrict__ xq, const float* __restrict__ xs,
            const int* __restrict__ xa, int32_t* __restrict__ dbg, int KS){
  constexpr int RG = 1;
  extern __shared__ __attribute__((aligned(16))) uint8_t kt_lds[];
  using F = KtFlat<KT_FMT_TERN, MT>;
  constexpr int UW = F::UW, UP = F::UP;
  const int NU = a.NU, S = kt_steps(NU), M = a.M;
  const int lane = threadIdx.x & 63, j = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), r = lane & 7, c = lane >> 3;
  uint8_t* xw = kt_lds + (size_t)j * MT * KT_KL * UP;               /* this wave's step: [MT][8 units][UP] */
  float* fv = (float*)(kt_lds + (size_t)S * MT * KT_KL * UP);       /* [RG][S][MT][64]: (float)(v - XA) */
  float* mv = fv + RG * S * MT * 64;                                /* [RG][S][MT][64]: XS d */

  /* the block's row groups are in one matrix (RG = 2: every matrix has an even number of row groups, the launcher
     checks) */
  const int g = RG * blockIdx.x;
  int mi = 0;
  if(a.nmat > 1 && g >= a.mat[1].rg0) mi = 1;
  if(a.nmat > 2 && g >= a.mat[2].rg0) mi = 2;
  const KtMat& m = a.mat[mi];
  const int rg0 = g - m.rg0, R = m.R;
  const uint4* wb = (const uint4*)m.codes;
  const uint16_t* sb = m.scales;
  const int u = j * KT_KL + c;
  const bool uok = u < NU;
  const int uu = uok ? u : 0;
  const unsigned o0 = uok ? (unsigned)kt_widx(NU, rg0, j, 0, c, r) : 0u;
  const unsigned o1 = uok ? (unsigned)kt_widx(NU, rg0, j, 1, c, r) : 0u;
  const unsigned os = uok ? (unsigned)kt_sidx(NU, rg0, u, r) : 0u;
  KtStep w[RG];
#pragma unroll
  for(int q = 0; q < RG; ++q){                                      /* row group rg0 + q: one row group further */
    w[q].c0 = kt_ldnt(wb + (long long)q * NU * 16 + o0);
    w[q].c1 = kt_ldnt(wb + (long long)q * NU * 16 + o1);
    w[q].hs = sb[(long long)q * NU * 8 + os];
  }
  const int nc = NU - j * KT_KL < KT_KL ? NU - j * KT_KL : KT_KL;
  const int o = lane * 16, oc = o < nc * UW ? o : 0;                /* the lane's 16 bytes of the step's row */
  for(int t0 = 0; t0 < M; t0 += MT){                               /* uniform */
    const int nt = min(MT, M - t0);
    uint4 stg[MT];
    uint32_t sa[2][MT];                                             /* unit scale (f32 bits), unit sum */
#pragma unroll
    for(int t = 0; t < MT; ++t){
      const int n = t0 + (t < nt ? t : 0);
      stg[t] = *(const uint4*)(xq + (long long)n * a.ldq + (long long)j * KT_KL * UW + oc);
      sa[0][t] = __float_as_uint(xs[(long long)n * a.ldxs + uu]);
      sa[1][t] = (uint32_t)xa[(long long)n * a.ldxs + uu];
    }
    kt_pin<MT>(&stg[0], &sa[0][0]);
#pragma unroll
    for(int t = 0; t < MT; ++t) *(uint4*)(xw + t * KT_KL * UP + (o / UW) * UP + o % UW) = stg[t];
    kt_wave_sync();
#pragma unroll
    for(int t = 0; t < MT; ++t){
      if(t < nt){                                                   /* uniform */
        int vv[2];
        const uint8_t* xrow = xw + (t * KT_KL + (uok ? c : 0)) * UP;
        if(RG == 2) kt_unit2_lds(w[0].c0, w[0].c1, w[1].c0, w[1].c1, xrow, vv);
        else vv[0] = kt_unit_lds<KT_FMT_TERN>(w[0].c0, w[0].c1, xrow);
#pragma unroll
        for(int q = 0; q < RG; ++q){
          const float d = uok ? kt_h2f(w[q].hs) : 0.0f;
          const int v = uok ? vv[q] - (int)sa[1][t] : 0;
          fv[((q * S + j) * MT + t) * 64 + lane] = (float)v;
          mv[((q * S + j) * MT + t) * 64 + lane] = __uint_as_float(sa[0][t]) * d;
          const int row = (rg0 + q) * KT_RG + r;
          if(DBG && uok && row < R) dbg[((long long)(t0 + t) * R + row) * NU + u] = v;
        }
      }
    }
    __syncthreads();
    if(j == 0){
#pragma unroll
      for(int q = 0; q < RG; ++q){
        float tot[MT];
#pragma unroll
        for(int t = 0; t < MT; ++t){
          tot[t] = 0.0f;
          for(int k = 0; k < KS; ++k){                              /* uniform */
            const int s_lo = k * S / KS, ns = (k + 1) * S / KS - s_lo;
            const int i0 = ((q * S + s_lo) * MT + t) * 64 + lane;
            float acc = fmaf(fv[i0], mv[i0], 0.0f);
            if(ns > 1) acc = fmaf(fv[i0 + MT * 64], mv[i0 + MT * 64], acc);
            const float y = kt_row_sum(acc);
            tot[t] = k == 0 ? y : tot[t] + y;
          }
        }
        const int row = (rg0 + q) * KT_RG + r;
        if(c == 0 && row < R){
#pragma unroll
          for(int t = 0; t < MT; ++t){
            if(a.hp){                                               /* rows 2t, 2t + 1 -> token t (MT even) */
              if(!(t & 1) && t < nt) m.y[(long long)((t0 + t) >> 1) * m.ldy + row] = tot[t] + tot[t + 1];
            } else if(t < nt) m.y[(long long)(t0 + t) * m.ldy + row] = tot[t];
          }
        }
      }
    }
    if(t0 + MT < M) __syncthreads();                                /* the next chunk rewrites the LDS */
  }
}

template __global__ void k_gemv_stepm<2, false>(const KtGemvArgs, const int8_t*, const float*, const int*, int32_t*, int);
template __global__ void k_gemv_stepm<2, true>(const KtGemvArgs, const int8_t*, const float*, const int*, int32_t*, int);
template __global__ void k_gemv_stepm<4, false>(const KtGemvArgs, const int8_t*, const float*, const int*, int32_t*, int);
template __global__ void k_gemv_stepm<4, true>(const KtGemvArgs, const int8_t*, const float*, const int*, int32_t*, int);
