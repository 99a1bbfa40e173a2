/* kt_gemv.h - the decode product of the quantized linear layer (k_tc_mv*, tc_hip.cu:180-240; lt_mv_q8,
   lightning.cu:258-284): ternary (kt2) or q8_0 (kq8) weights against 1 .. 16 int8 token rows.

   One wave per 8-row group, each row's K units spread over 8 lanes (lane = 8 c + r takes units c, c + 8, ... of
   row r), optionally several waves per row group taking K slices. A wave streams its rows with 128-bit loads (1 KB
   contiguous per instruction) running a register batch ahead of their use. Ternary digits are isolated with one
   AND per 4 columns (slots 0..2 keep their 4^k factor and are shifted back exactly after the unit; slot 3 takes one
   shift), so a unit costs 8 x (4 dot4 + 5 logic ops) per lane, independent of the trit values. Explicit
   instantiations are spread over kt_gemv_*.hip so the library compiles in parallel. */
#pragma once
#include "kt_common.h"

/* ------------------------------------------------------------------ the product */
/* the exact value of one unit of one row: m = the row's masked digit words (ternary) or int8 words (q8_0), x = the
   unit's activation words */
template <int FMT>
__device__ __forceinline__ int kt_unit(const uint32_t m[4][8], const int x[32]){
  if(FMT == KT_FMT_TERN){
    int a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
    for(int j = 0; j < 8; ++j){
      a0 = kt_dot4((int)m[0][j], x[4 * j + 0], a0);
      a1 = kt_dot4((int)m[1][j], x[4 * j + 1], a1);
      a2 = kt_dot4((int)m[2][j], x[4 * j + 2], a2);
      a0 = kt_dot4((int)m[3][j], x[4 * j + 3], a0);
    }
    return a0 + (a1 >> 2) + (a2 >> 4);                      /* slots 1, 2 carry 4, 16: exact shifts */
  } else {
    int a = 0;
#pragma unroll
    for(int j = 0; j < 8; ++j) a = kt_dot4((int)m[0][j], x[j], a);
    return a;
  }
}

template <int FMT>
__device__ __forceinline__ void kt_split_words(const uint4 c0, const uint4 c1, uint32_t m[4][8]){
  const uint32_t w[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
  for(int j = 0; j < 8; ++j){
    if(FMT == KT_FMT_TERN){
      m[0][j] = w[j] & 0x03030303u;
      m[1][j] = w[j] & 0x0C0C0C0Cu;
      m[2][j] = w[j] & 0x30303030u;
      m[3][j] = (w[j] >> 6) & 0x03030303u;
    } else {
      m[0][j] = w[j];
    }
  }
}

/* the fixed xor butterfly over the 8 k-lanes of a row (lane bits 3..5): every lane ends with the same value */
__device__ __forceinline__ float kt_row_sum(float v){
  v += __shfl_xor(v, 8);
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

/* one batch of UB steps of a wave: the rows' code words and scales (loads only: issued ahead of their use) */
struct KtBatch {
  uint4 c0[KT_UB], c1[KT_UB];
  uint16_t hs[KT_UB];
};

__device__ __forceinline__ void kt_load_batch(KtBatch& b, const uint4* __restrict__ wb, const uint16_t* __restrict__ sb,
                                              int NU, int rg, int s0, int s1, int c, int r){
#pragma unroll
  for(int k = 0; k < KT_UB; ++k){
    const int u = (s0 + k) * KT_KL + c;
    if(s0 + k < s1 && u < NU){
      b.c0[k] = kt_ldnt(wb + kt_widx(NU, rg, s0 + k, 0, c, r));
      b.c1[k] = kt_ldnt(wb + kt_widx(NU, rg, s0 + k, 1, c, r));
      b.hs[k] = sb[kt_sidx(NU, rg, u, r)];
    }
  }
}

/* a unit's activation words of token slot t: from the LDS staging (XL) or through L1 */
template <int FMT, bool XL>
__device__ __forceinline__ void kt_get_x(const uint8_t* xl, int NU, int t, int u, const int8_t* __restrict__ xq,
                                         long long ldq, int n, int x[32]){
  constexpr int UW = FMT == KT_FMT_TERN ? 128 : 32, UP = UW + 16;
  const uint4* q = XL ? (const uint4*)(xl + ((size_t)t * NU + u) * UP) : (const uint4*)(xq + n * ldq + (long long)u * UW);
#pragma unroll
  for(int j = 0; j < UW / 16; ++j){
    const uint4 v = q[j];
    x[4 * j] = (int)v.x; x[4 * j + 1] = (int)v.y; x[4 * j + 2] = (int)v.z; x[4 * j + 3] = (int)v.w;
  }
}

template <int FMT, int MT, bool XL>
__device__ __forceinline__ void kt_compute_batch(const KtBatch& b, int NU, int s0, int s1, int c, int row, int R,
                                                 int t0, int nt, const uint8_t* xl, const float* sl, const int* al,
                                                 const int8_t* __restrict__ xq, long long ldq,
                                                 const float* __restrict__ xs, const int* __restrict__ xa, int ldxs,
                                                 int32_t* __restrict__ dbg, float acc[MT]){
#pragma unroll
  for(int k = 0; k < KT_UB; ++k){
    const int u = (s0 + k) * KT_KL + c;
    if(s0 + k < s1 && u < NU){
      const float d = kt_h2f(b.hs[k]);
      uint32_t m[4][8];
      kt_split_words<FMT>(b.c0[k], b.c1[k], m);
#pragma unroll
      for(int t = 0; t < MT; ++t){
        if(t < nt){
          const int n = t0 + t;
          int x[32];
          kt_get_x<FMT, XL>(xl, NU, t, u, xq, ldq, n, x);
          int v = kt_unit<FMT>(m, x);
          const float s = XL ? sl[t * NU + u] : xs[(long long)n * ldxs + u];
          if(FMT == KT_FMT_TERN) v -= XL ? al[t * NU + u] : xa[(long long)n * ldxs + u];
          acc[t] = fmaf((float)v, FMT == KT_FMT_TERN ? s * d : d * s, acc[t]);
          if(dbg && row < R) dbg[((long long)n * R + row) * NU + u] = v;
        }
      }
    }
  }
}

/* one step of one lane: its unit's two code loads and scale */
struct KtStep {
  uint4 c0, c1;
  uint16_t hs;
};

template <int FMT, int MT, bool DBG>
__device__ __forceinline__ void kt_compute_step(const KtStep& st, bool valid, int NU, int u, int row, int R, int t0,
                                                int nt, const uint8_t* xl, const float* sl, const int* al,
                                                int32_t* __restrict__ dbg, float acc[MT]){
  /* branch-free: an invalid step reads unit 0 of the staging and adds fmaf(0, 0, acc) = acc */
  constexpr int UW = FMT == KT_FMT_TERN ? 128 : 32, UP = UW + 16;
  const int uu = valid ? u : 0;
  const float d = valid ? kt_h2f(st.hs) : 0.0f;
  uint32_t m[4][8];
  kt_split_words<FMT>(st.c0, st.c1, m);
#pragma unroll
  for(int t = 0; t < MT; ++t){
    if(t < nt){
      int x[32];
      const uint4* q = (const uint4*)(xl + ((size_t)t * NU + uu) * UP);
#pragma unroll
      for(int j = 0; j < UW / 16; ++j){
        const uint4 v = q[j];
        x[4 * j] = (int)v.x; x[4 * j + 1] = (int)v.y; x[4 * j + 2] = (int)v.z; x[4 * j + 3] = (int)v.w;
      }
      int v = kt_unit<FMT>(m, x);
      const float s = sl[t * NU + uu];
      if(FMT == KT_FMT_TERN) v -= al[t * NU + uu];
      v = valid ? v : 0;
      acc[t] = fmaf((float)v, FMT == KT_FMT_TERN ? s * d : d * s, acc[t]);
      if(DBG && valid && row < R) dbg[((long long)(t0 + t) * R + row) * NU + u] = v;
    }
  }
}

/* The plain product for 8 .. 16 tokens (or widths whose staging does not fit in LDS): grid (ceil(row groups /
   RGB), npass), block 64 KS RGB. Wave (rgl, ks) takes row group blockIdx.x RGB + rgl and the K slice ks of KS
   (steps [ks S / KS, (ks + 1) S / KS)). The same lanes, arithmetic and summation order as k_gemv_pipe; the
   activations are read through L1 (XL = false) or from an LDS staging (XL); the weight loads run one register batch
   ahead (two batches, ping-pong). */
template <int FMT, int MT, int KS, int RGB, bool XL>
__global__ void __launch_bounds__(64 * KS * RGB) k_gemv(const KtGemvArgs a, const int8_t* __restrict__ xq,
                                                        const float* __restrict__ xs, const int* __restrict__ xa,
                                                        int32_t* __restrict__ dbg){
  extern __shared__ __attribute__((aligned(16))) uint8_t kt_lds[];
  constexpr int UW = FMT == KT_FMT_TERN ? 128 : 32, UP = UW + 16, W = KS * RGB;
  const int NU = a.NU, S = kt_steps(NU);
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rgl = wv / KS, ks = wv % KS, r = lane & 7, c = lane >> 3;
  const int g = blockIdx.x * RGB + rgl, t0 = blockIdx.y * MT, nt = min(MT, a.M - t0);
  int mi = 0;
  if(a.nmat > 1 && g >= a.mat[1].rg0) mi = 1;
  if(a.nmat > 2 && g >= a.mat[2].rg0) mi = 2;
  const KtMat mat = a.mat[mi];
  const int rg = g - mat.rg0, row = rg * KT_RG + r;
  const int ngroups = a.mat[a.nmat - 1].rg0 + kt_r8(a.mat[a.nmat - 1].R);
  const bool live = g < ngroups;
  const int s_lo = ks * S / KS, s_hi = (ks + 1) * S / KS;
  const uint4* __restrict__ wb = (const uint4*)mat.codes;
  const uint16_t* __restrict__ sb = mat.scales;
  uint8_t* xl = kt_lds;                                        /* [MT][NU][UP] (XL) */
  float* sl = (float*)(kt_lds + (XL ? (size_t)MT * NU * UP : 0));   /* [MT][NU] */
  int* al = (int*)(sl + (XL ? MT * NU : 0));                   /* [MT][NU] (ternary) */
  float* red = (float*)(al + (XL && FMT == KT_FMT_TERN ? MT * NU : 0));   /* [W][MT][8] */

  KtBatch A, B;
  if(live) kt_load_batch(A, wb, sb, NU, rg, s_lo, s_hi, c, r);
  if(XL){
    const int nchunk = nt * NU * (UW / 16);
    for(int i = threadIdx.x; i < nchunk; i += 64 * W){
      const int t = i / (NU * (UW / 16)), rem = i - t * NU * (UW / 16), u = rem / (UW / 16), k = rem % (UW / 16);
      *(uint4*)(xl + ((size_t)t * NU + u) * UP + 16 * k) =
          *(const uint4*)(xq + (long long)(t0 + t) * a.ldq + (long long)u * UW + 16 * k);
    }
    for(int i = threadIdx.x; i < nt * NU; i += 64 * W){
      const int t = i / NU, u = i - t * NU;
      sl[i] = xs[(long long)(t0 + t) * a.ldxs + u];
      if(FMT == KT_FMT_TERN) al[i] = xa[(long long)(t0 + t) * a.ldxs + u];
    }
    __syncthreads();
  }

  float acc[MT];
#pragma unroll
  for(int t = 0; t < MT; ++t) acc[t] = 0.0f;
  if(live){
    for(int s0 = s_lo; s0 < s_hi; s0 += 2 * KT_UB){
      if(s0 + KT_UB < s_hi) kt_load_batch(B, wb, sb, NU, rg, s0 + KT_UB, s_hi, c, r);
      kt_compute_batch<FMT, MT, XL>(A, NU, s0, s_hi, c, row, mat.R, t0, nt, xl, sl, al, xq, a.ldq, xs, xa, a.ldxs,
                                    dbg, acc);
      if(s0 + 2 * KT_UB < s_hi) kt_load_batch(A, wb, sb, NU, rg, s0 + 2 * KT_UB, s_hi, c, r);
      if(s0 + KT_UB < s_hi)
        kt_compute_batch<FMT, MT, XL>(B, NU, s0 + KT_UB, s_hi, c, row, mat.R, t0, nt, xl, sl, al, xq, a.ldq, xs, xa,
                                      a.ldxs, dbg, acc);
    }
  }
  float y[MT];
#pragma unroll
  for(int t = 0; t < MT; ++t) y[t] = kt_row_sum(acc[t]);
  if(KS > 1){
    if(c == 0){
#pragma unroll
      for(int t = 0; t < MT; ++t) red[(wv * MT + t) * 8 + r] = y[t];
    }
    __syncthreads();
    if(ks != 0) return;
#pragma unroll
    for(int t = 0; t < MT; ++t){
      float v = red[((rgl * KS) * MT + t) * 8 + r];
#pragma unroll
      for(int k = 1; k < KS; ++k) v += red[((rgl * KS + k) * MT + t) * 8 + r];
      y[t] = v;
    }
  }
  if(!live) return;
#pragma unroll
  for(int t = 0; t < MT; ++t)
    if(c == 0 && t < nt && row < mat.R) mat.y[(long long)(t0 + t) * mat.ldy + row] = y[t];
}

#ifndef KT_PF
#define KT_PF 2                       /* steps a wave's weight loads run ahead of their use */
#endif

/* The pipelined product (activations staged in LDS): grid (items, npass), block 64 KS. Block b takes the RPL row
   groups b RPL .. b RPL + RPL - 1 (a lane takes its unit of all of them, so one read of the staged activations
   serves RPL rows); wave ks of the block the K slice ks of KS (steps [ks S / KS, (ks + 1) S / KS)). The loads of
   step f + KT_PF are issued when step f is used, into a ring of KT_PF register sets (the loop is unrolled by
   KT_PF); every step issues its loads unconditionally (a step past the slice or the matrix reads the first 16 bytes
   of the codes, one cache line for the wave) and only the compute is skipped, by a wave-uniform branch, so the
   compiler's wait counts stay exact and the loads of later steps stay in flight. A lane chains its units of the
   slice in order; the row's 8 lanes are added by the xor butterfly; the KS slices of a row in slice order in LDS.
   The activations of the whole width (MT tokens) are staged in LDS once per block, a unit's int8 values at a
   stride padded by 16 bytes (the 8 units a ds_read_b128 touches fall on disjoint banks), after the first weight
   loads are issued. DBG: also store every unit's exact value (a separate instantiation). */
template <int RPL>
struct KtStepR { KtStep row[RPL]; };

template <int FMT, int MT, int KS, int RPL, bool DBG>
__global__ void __launch_bounds__(64 * KS) k_gemv_pipe(const KtGemvArgs a, const int8_t* __restrict__ xq,
                                                       const float* __restrict__ xs, const int* __restrict__ xa,
                                                       int32_t* __restrict__ dbg){
  extern __shared__ __attribute__((aligned(16))) uint8_t kt_lds[];
  constexpr int UW = FMT == KT_FMT_TERN ? 128 : 32, UP = UW + 16, D = KT_PF;
  const int NU = a.NU, S = kt_steps(NU);
  const int lane = threadIdx.x & 63, ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), r = lane & 7, c = lane >> 3;
  const int t0 = blockIdx.y * MT, nt = min(MT, a.M - t0);
  const int ngroups = a.mat[a.nmat - 1].rg0 + kt_r8(a.mat[a.nmat - 1].R);
  const int g0 = (int)blockIdx.x * RPL;
  const int s_lo = ks * S / KS, ns = (ks + 1) * S / KS - s_lo;  /* this slice's steps */
  uint8_t* xl = kt_lds;                                        /* [MT][NU][UP] */
  float* sl = (float*)(kt_lds + (size_t)MT * NU * UP);         /* [MT][NU] */
  int* al = (int*)(sl + MT * NU);                              /* [MT][NU] (ternary) */
  float* red = (float*)(al + (FMT == KT_FMT_TERN ? MT * NU : 0));   /* [KS][RPL][MT][8] */
  const uint4* __restrict__ dummy = (const uint4*)a.mat[0].codes;

  auto matrix = [&](int g) -> const KtMat& {
    int mi = 0;
    if(a.nmat > 1 && g >= a.mat[1].rg0) mi = 1;
    if(a.nmat > 2 && g >= a.mat[2].rg0) mi = 2;
    return a.mat[mi];
  };
  /* the loads of step f of the RPL row groups, unconditionally */
  auto load_step = [&](KtStepR<RPL>& st, int f){
    const int s = s_lo + f, u = s * KT_KL + c;
#pragma unroll
    for(int j = 0; j < RPL; ++j){
      const int g = g0 + j;
      const bool ok = f < ns && g < ngroups && u < NU;
      const KtMat& m = matrix(g < ngroups ? g : 0);
      const int rg = g - m.rg0;
      const uint4* p0 = ok ? (const uint4*)m.codes + kt_widx(NU, rg, s, 0, c, r) : dummy;
      const uint4* p1 = ok ? (const uint4*)m.codes + kt_widx(NU, rg, s, 1, c, r) : dummy;
      const uint16_t* ps = ok ? m.scales + kt_sidx(NU, rg, u, r) : (const uint16_t*)dummy;
      st.row[j].c0 = kt_ldnt(p0);
      st.row[j].c1 = kt_ldnt(p1);
      st.row[j].hs = *ps;
    }
  };

  KtStepR<RPL> ring[D];
#pragma unroll
  for(int k = 0; k < D; ++k) load_step(ring[k], k);
  {
    const int nchunk = nt * NU * (UW / 16);
    for(int i = threadIdx.x; i < nchunk; i += 64 * KS){
      const int t = i / (NU * (UW / 16)), rem = i - t * NU * (UW / 16), u = rem / (UW / 16), k = rem % (UW / 16);
      *(uint4*)(xl + ((size_t)t * NU + u) * UP + 16 * k) =
          *(const uint4*)(xq + (long long)(t0 + t) * a.ldq + (long long)u * UW + 16 * k);
    }
    for(int i = threadIdx.x; i < nt * NU; i += 64 * KS){
      const int t = i / NU, u = i - t * NU;
      sl[i] = xs[(long long)(t0 + t) * a.ldxs + u];
      if(FMT == KT_FMT_TERN) al[i] = xa[(long long)(t0 + t) * a.ldxs + u];
    }
    __syncthreads();
  }

  float acc[RPL][MT];
#pragma unroll
  for(int j = 0; j < RPL; ++j)
#pragma unroll
    for(int t = 0; t < MT; ++t) acc[j][t] = 0.0f;
  for(int f0 = 0; f0 < ns; f0 += D){
#pragma unroll
    for(int k = 0; k < D; ++k){
      const int f = f0 + k;
      if(f < ns){                                              /* wave-uniform */
        const int u = (s_lo + f) * KT_KL + c;
        const int uu = u < NU ? u : 0;
        const bool uok = u < NU;
#pragma unroll
        for(int t = 0; t < MT; ++t){
          if(t < nt){
            int x[32];
            const uint4* q = (const uint4*)(xl + ((size_t)t * NU + uu) * UP);
#pragma unroll
            for(int jj = 0; jj < UW / 16; ++jj){
              const uint4 v = q[jj];
              x[4 * jj] = (int)v.x; x[4 * jj + 1] = (int)v.y; x[4 * jj + 2] = (int)v.z; x[4 * jj + 3] = (int)v.w;
            }
            const float s = sl[t * NU + uu];
            const int xsum = FMT == KT_FMT_TERN ? al[t * NU + uu] : 0;
#pragma unroll
            for(int j = 0; j < RPL; ++j){
              const KtStep& st = ring[k].row[j];
              uint32_t m[4][8];
              kt_split_words<FMT>(st.c0, st.c1, m);
              int v = kt_unit<FMT>(m, x) - xsum;
              const float dd = uok ? kt_h2f(st.hs) : 0.0f;
              v = uok ? v : 0;
              acc[j][t] = fmaf((float)v, FMT == KT_FMT_TERN ? s * dd : dd * s, acc[j][t]);
              if(DBG && uok){
                const int g = g0 + j;
                if(g < ngroups){
                  const KtMat& mm = matrix(g);
                  const int row = (g - mm.rg0) * KT_RG + r;
                  if(row < mm.R) dbg[((long long)(t0 + t) * mm.R + row) * NU + u] = v;
                }
              }
            }
          }
        }
      }
      load_step(ring[k], f + D);
    }
  }
  float y[RPL][MT];
#pragma unroll
  for(int j = 0; j < RPL; ++j)
#pragma unroll
    for(int t = 0; t < MT; ++t) y[j][t] = kt_row_sum(acc[j][t]);
  if(KS > 1){
    if(c == 0){
#pragma unroll
      for(int j = 0; j < RPL; ++j)
#pragma unroll
        for(int t = 0; t < MT; ++t) red[((ks * RPL + j) * MT + t) * 8 + r] = y[j][t];
    }
    __syncthreads();
    if(ks != 0) return;
#pragma unroll
    for(int j = 0; j < RPL; ++j)
#pragma unroll
      for(int t = 0; t < MT; ++t){
        float v = red[((0 * RPL + j) * MT + t) * 8 + r];
#pragma unroll
        for(int kk = 1; kk < KS; ++kk) v += red[((kk * RPL + j) * MT + t) * 8 + r];
        y[j][t] = v;
      }
  }
  if(c != 0) return;
#pragma unroll
  for(int j = 0; j < RPL; ++j){
    const int g = g0 + j;
    if(g < ngroups){
      const KtMat& mat = matrix(g);
      const int row = (g - mat.rg0) * KT_RG + r;
#pragma unroll
      for(int t = 0; t < MT; ++t)
        if(t < nt && row < mat.R) mat.y[(long long)(t0 + t) * mat.ldy + row] = y[j][t];
    }
  }
}
