/* kt_gemv.h - the decode product with one load round trip per wave (k_tc_mv*, tc_hip.cu:180-240; lt_mv_q8,
   lightning.cu:258-284): ternary (kt2) or q8_0 (kq8) weights against any number of int8 token rows.

   Grid: one block per row group (8 rows) over all matrices of the launch; block: KS waves, wave ks takes the K slice
   of steps [ks S / KS, (ks + 1) S / KS) (KS = kt_kslices: at most KT_SL steps a slice up to 16 slices). A wave issues
   the code and scale loads of its whole slice at once (for slices of <= KT_SL steps: one memory round trip), then
   serves every token with them: tokens go in chunks of MT; a chunk's activations of the slice are staged by the
   wave into its own LDS region (no block barrier), each lane (8 c + r) chains its units of the slice in order, the
   8 lanes of a row are added by the xor butterfly and the KS slices in slice order, in LDS, by wave 0. The tree is a
   function of C only, so a token's bits do not depend on M or on the other matrices of the launch.
   Loads are unconditional (a unit past the matrix reads the first 16 bytes of the codes) and only compute is
   skipped, by wave-uniform branches, so the compiler's wait counts stay exact. */
#pragma once
#ifndef KT_FLAT1_ONE
#define KT_FLAT1_ONE 1                /* one-token dense ternary k_gemv_flat1: activations first (kt_gemv_one_body) */
#endif
#include "kt_common.h"

#ifdef KT_TRACE                        /* a timeline build: per-block s_memrealtime stamps, one buffer per source file */
static __device__ unsigned long long kt_trace_buf[1 << 16];
static __device__ int kt_trace_on;
#define KT_GTS(k) do { if(kt_trace_on && threadIdx.x == 0 && blockIdx.x < 8192) \
    kt_trace_buf[blockIdx.x * 4 + (k)] = __builtin_amdgcn_s_memrealtime(); } while(0)
#else
#define KT_GTS(k) do {} while(0)
#endif

/* the fixed xor butterfly over the 8 k-lanes of a row (lane bits 3..5): every lane ends with the same value (each
   adds the same pair); the exchanges run on the VALU (kf_xor) */
__device__ __forceinline__ float kt_row_sum(float v){
  v += kf_xorf<8>(v);
  v += kf_xorf<16>(v);
  v += kf_xorf<32>(v);
  return v;
}

/* one step of one lane: its unit's two code loads and scale */
struct KtStep {
  uint4 c0, c1;
  uint16_t hs;
};


/* the exact value of one unit from its two code words and its staged activations (LDS), half by half. Ternary:
   (w >> 2k) & 0x03030303 is the digit vector (t + 1) of columns 4 k' .. of the word, so slot 0 and slot 3 (shifted
   down first) go to a0, slot 1 to a1 and slot 2 to a2 unshifted, where they carry the exact factors 4 and 16 that
   the final shifts remove; the unit's sum of digits times activations, minus XA, is then sum t q. q8_0: one dot4
   per word. Integer arithmetic, so the order inside a unit is free. */
template <int FMT>
__device__ __forceinline__ int kt_unit_lds(const uint4 c0, const uint4 c1, const uint8_t* xrow){
  const uint4* q = (const uint4*)xrow;
  if(FMT == KT_FMT_TERN){
    int a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
    for(int h = 0; h < 2; ++h){
      const uint4 cw = h ? c1 : c0;
      const uint32_t ww[4] = {cw.x, cw.y, cw.z, cw.w};
#pragma unroll
      for(int j = 0; j < 4; ++j){
        const uint4 x = q[4 * h + j];
        a0 = kt_dot4((int)(ww[j] & 0x03030303u), (int)x.x, a0);
        a1 = kt_dot4((int)(ww[j] & 0x0C0C0C0Cu), (int)x.y, a1);
        a2 = kt_dot4((int)(ww[j] & 0x30303030u), (int)x.z, a2);
        a0 = kt_dot4((int)((ww[j] >> 6) & 0x03030303u), (int)x.w, a0);
      }
    }
    return a0 + (a1 >> 2) + (a2 >> 4);
  } else {
    const uint4 x0 = q[0], x1 = q[1];
    int a = kt_dot4((int)c0.x, (int)x0.x, 0);
    a = kt_dot4((int)c0.y, (int)x0.y, a);
    a = kt_dot4((int)c0.z, (int)x0.z, a);
    a = kt_dot4((int)c0.w, (int)x0.w, a);
    a = kt_dot4((int)c1.x, (int)x1.x, a);
    a = kt_dot4((int)c1.y, (int)x1.y, a);
    a = kt_dot4((int)c1.z, (int)x1.z, a);
    return kt_dot4((int)c1.w, (int)x1.w, a);
  }
}

/* an empty asm that takes every staged row word (q, N of them) and every unit scale and sum (w, 2 N): the loads
   that produce them are all issued before it, with one wait for all, instead of each load sunk to its own use */
template <int N>
__device__ __forceinline__ void kt_pin(uint4* v, uint32_t* w){
  kt_u32x4* q = (kt_u32x4*)v;
  if(N == 1) asm("" : "+v"(q[0]), "+v"(w[0]), "+v"(w[1]));
  else if(N == 2) asm("" : "+v"(q[0]), "+v"(q[1]), "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]));
  else if(N == 3) asm("" : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]), "+v"(w[4]), "+v"(w[5]));
  else if(N == 4) asm("" : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3]), "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]), "+v"(w[4]), "+v"(w[5]), "+v"(w[6]), "+v"(w[7]));
  else if(N == 6) asm("" : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3]), "+v"(q[4]), "+v"(q[5]), "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]), "+v"(w[4]), "+v"(w[5]), "+v"(w[6]), "+v"(w[7]), "+v"(w[8]), "+v"(w[9]), "+v"(w[10]), "+v"(w[11]));
  else if(N == 8) asm("" : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3]), "+v"(q[4]), "+v"(q[5]), "+v"(q[6]), "+v"(q[7]), "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]), "+v"(w[4]), "+v"(w[5]), "+v"(w[6]), "+v"(w[7]), "+v"(w[8]), "+v"(w[9]), "+v"(w[10]), "+v"(w[11]), "+v"(w[12]), "+v"(w[13]), "+v"(w[14]), "+v"(w[15]));
}

/* kt_q8_quant's numbers for the 8 lanes of one 32-column unit (lane bits 0..2 = r: floats 4 r .. 4 r + 3 of the
   unit): relu^2 first when RELU; amax by three VALU exchanges (exact in any order); q = rne(v 127 / amax) packed
   little-endian; d = fp16(amax / 127) as f32 (llama.cpp's CPU q8_0 rounding, lt_quant2 lightning.cu:470) */
template <bool RELU>
__device__ __forceinline__ uint32_t kt_q8_unit_quant(const uint4 raw, float& d){
  float v[4] = {__uint_as_float(raw.x), __uint_as_float(raw.y), __uint_as_float(raw.z), __uint_as_float(raw.w)};
  float a = 0.0f;
#pragma unroll
  for(int i = 0; i < 4; ++i){
    if(RELU){ v[i] = fmaxf(v[i], 0.0f); v[i] = v[i] * v[i]; }
    a = fmaxf(a, fabsf(v[i]));
  }
  a = fmaxf(a, kf_xorf<1>(a));
  a = fmaxf(a, kf_xorf<2>(a));
  a = fmaxf(a, kf_xorf<4>(a));
  const float id = a != 0.0f ? 127.0f / a : 0.0f;
  uint32_t q = 0;
#pragma unroll
  for(int i = 0; i < 4; ++i) q |= (uint32_t)(uint8_t)(int8_t)__float2int_rn(v[i] * id) << (8 * i);
  d = __half2float(__float2half_rn(a / 127.0f));
  return q;
}

/* the slice sums p[0], p[st], p[2 st], ... (KS <= 16 of them) added left to right, every LDS read issued before the
   first add (a select, not a +0, past the last slice keeps the sum exact) */
__device__ __forceinline__ float kt_slice_sum(const float* p, int st, int KS){
  float t[KT_KSMAX];
#pragma unroll
  for(int q = 0; q < KT_KSMAX; ++q) t[q] = p[(q < KS ? q : 0) * st];
  float v = t[0];
#pragma unroll
  for(int q = 1; q < KT_KSMAX; ++q) v = q < KS ? v + t[q] : v;
  return v;
}

__device__ __forceinline__ void kt_wave_sync(){
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

template <int FMT, int MT, bool DBG, bool GRP>
__device__ __forceinline__ void kt_gemv_flat_body(const KtGemvArgs& a, const KtGroupedArgs& ga,
                                                  const int8_t* __restrict__ xq, const float* __restrict__ xs,
                                                  const int* __restrict__ xa, int32_t* __restrict__ dbg, int KS){
  extern __shared__ __attribute__((aligned(16))) uint8_t kt_lds[];
  using F = KtFlat<FMT, MT>;
  constexpr int UW = F::UW, UP = F::UP, SL = KT_SL;
  constexpr bool XF = FMT == KT_FMT_Q8X || FMT == KT_FMT_Q8R;         /* activations quantized here from fp32 */
  constexpr int WF = XF ? KT_FMT_Q8 : FMT;                           /* the weights' format */
  const int NU = GRP ? ga.NU : a.NU, S = kt_steps(NU);
  const int lane = threadIdx.x & 63, ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), r = lane & 7, c = lane >> 3;
  const int g = blockIdx.x;
  KT_GTS(0);
  /* the job of this block: a matrix's row group and its token rows. Dense: row group g of the launch's matrices,
     tokens 0 .. M - 1, output row t. Grouped (MoE): row group g of active expert act[blockIdx.y], the tokens of its
     list (entries off .. off + cnt - 1, input row xrow[p] or p), output row = entry p. */
  const uint4* __restrict__ wb;
  const uint16_t* __restrict__ sb;
  float* yout;
  int R, ldy, rg, M, p0, ldq, ldxs;
  const int* xrow = nullptr;
  if(GRP){
    /* the active count and this block's expert loaded together (act holds E entries: an index past the count reads
       an unused entry, not used) */
    const int nact = *ga.nact, e = ga.act[blockIdx.y];
    if((int)blockIdx.y >= nact) return;
    const uint8_t* base = ga.wexp[e];
    wb = (const uint4*)base;
    sb = (const uint16_t*)(base + (long long)kt_r8(ga.R) * NU * 256);
    R = ga.R; ldy = ga.ldy; rg = g; M = ga.cnt[e]; p0 = ga.off[e]; xrow = ga.xrow; ldq = ga.ldq; ldxs = ga.ldd;
    yout = ga.y;
  } else {
    int mi = 0;
    if(a.nmat > 1 && g >= a.mat[1].rg0) mi = 1;
    if(a.nmat > 2 && g >= a.mat[2].rg0) mi = 2;
    const KtMat& m = a.mat[mi];
    wb = (const uint4*)m.codes;
    sb = m.scales;
    R = m.R; ldy = m.ldy; rg = g - m.rg0; M = a.M; p0 = 0; ldq = a.ldq; ldxs = a.ldxs;
    yout = m.y;
  }
  const int row = rg * KT_RG + r;
  const int s_lo = ks * S / KS, ns = (ks + 1) * S / KS - s_lo;      /* this slice's steps (>= 1) */
  uint8_t* xw = kt_lds + (size_t)ks * F::XW;                         /* [MT][SL][8][UP] */
  float* red = (float*)(kt_lds + (size_t)KS * F::XW);                /* [KS][MT][8] */
  const bool one = ns <= SL;                                         /* wave-uniform */

  KtStep w[SL];
  /* every offset first (an integer select: a unit past the slice or the matrix reads offset 0), then every load,
     so no load waits for another */
  auto load_w = [&](int f0){
    unsigned o0[SL], o1[SL], os[SL];
#pragma unroll
    for(int j = 0; j < SL; ++j){
      const int f = f0 + j, s = s_lo + f, u = s * KT_KL + c;
      const bool ok = f < ns && u < NU;
      o0[j] = ok ? (unsigned)kt_widx(NU, rg, s, 0, c, r) : 0u;
      o1[j] = ok ? (unsigned)kt_widx(NU, rg, s, 1, c, r) : 0u;
      os[j] = ok ? (unsigned)kt_sidx(NU, rg, u, r) : 0u;
    }
#pragma unroll
    for(int j = 0; j < SL; ++j){
      w[j].c0 = kt_ldnt(wb + o0[j]);
      w[j].c1 = kt_ldnt(wb + o1[j]);
      w[j].hs = sb[os[j]];
    }
  };
  if(one) load_w(0);

  for(int t0 = 0; t0 < M; t0 += MT){
    const int nt = min(MT, M - t0);
    float acc[MT];
#pragma unroll
    for(int t = 0; t < MT; ++t) acc[t] = 0.0f;
    for(int f0 = 0; f0 < ns; f0 += SL){
      if(!one) load_w(f0);
      /* this chunk's activations: staged rows of the slice's steps, and the lane's unit scale and sum */
      uint32_t sa[2][SL][MT];                                        /* unit scale (f32 bits) and sum */
      uint4 stg[SL][MT];
      const int o = lane * 16;                                       /* the lane's 16 bytes of a step's row */
#pragma unroll
      for(int j = 0; j < SL; ++j){
        const int f = f0 + j, s = s_lo + (f < ns ? f : 0), u = s * KT_KL + c, uu = (f < ns && u < NU) ? u : 0;
        const int nc = NU - s * KT_KL < KT_KL ? NU - s * KT_KL : KT_KL;
#pragma unroll
        for(int t = 0; t < MT; ++t){
          const int pe = p0 + t0 + (t < nt ? t : 0), n = xrow ? xrow[pe] : pe;
          if(XF){
            /* 4 floats a lane: unit c = lane / 8 of the step, floats 4 r .. (lanes of a unit past a ragged step read
               the step's first floats; that unit is never used) */
            const int of = lane * 4, ofc = of < nc * 32 ? of : 0;
            sa[0][j][t] = 0u;
            sa[1][j][t] = 0u;
            stg[j][t] = *(const uint4*)(ga.xf + (long long)n * ga.ldxf + (long long)s * KT_KL * 32 + ofc);
          } else {
            (void)uu;
            sa[0][j][t] = __float_as_uint(xs[(long long)n * ldxs + uu]);
            sa[1][j][t] = FMT == KT_FMT_TERN ? (uint32_t)xa[(long long)n * ldxs + uu] : 0u;
            const int oc = o < nc * UW ? o : 0;
            stg[j][t] = *(const uint4*)(xq + (long long)n * ldq + (long long)s * KT_KL * UW + oc);
          }
        }
      }
      kt_pin<SL * MT>(&stg[0][0], &sa[0][0][0]);                                  /* every load above is issued before a write */
#ifdef KT_TRACE
      { uint32_t sink = 0;
#pragma unroll
        for(int jj = 0; jj < SL; ++jj) sink ^= w[jj].c0.x ^ w[jj].c1.y;
        if(sink == 0x12345u && threadIdx.x == 1) kt_trace_buf[65535] = 1; }
      KT_GTS(1);
#endif
      /* unconditional writes: a slot of a unit, step or token that does not exist is never read; q8_0 rows are 256
         bytes a step, so lanes past them write the wave's dump slot */
      if(XF){
        /* the lane's 4 bytes of unit c at byte 4 r, and the unit's scale (every lane of the unit has it: the lanes
           that use unit c are exactly these) */
#pragma unroll
        for(int j = 0; j < SL; ++j)
#pragma unroll
          for(int t = 0; t < MT; ++t){
            float d;
            const uint32_t q = kt_q8_unit_quant<FMT == KT_FMT_Q8R>(stg[j][t], d);
            *(uint32_t*)(xw + ((t * SL + j) * KT_KL + c) * UP + 4 * r) = q;
            sa[0][j][t] = __float_as_uint(d);
          }
      } else {
        const bool in = o < KT_KL * UW;
        const int lo = (o / UW) * UP + o % UW;
#pragma unroll
        for(int j = 0; j < SL; ++j)
#pragma unroll
          for(int t = 0; t < MT; ++t)
            *(uint4*)(xw + (in ? (t * SL + j) * KT_KL * UP + lo : F::XW - 16)) = stg[j][t];
      }
      kt_wave_sync();
#pragma unroll
      for(int j = 0; j < SL; ++j){
        const int f = f0 + j, u = (s_lo + f) * KT_KL + c;
        if(f < ns){                                                  /* wave-uniform */
          const bool uok = u < NU;
          const float d = uok ? kt_h2f(w[j].hs) : 0.0f;
#pragma unroll
          for(int t = 0; t < MT; ++t){
            if(t < nt){
              int v = kt_unit_lds<WF>(w[j].c0, w[j].c1, xw + ((t * SL + j) * KT_KL + (uok ? c : 0)) * UP) - (int)sa[1][j][t];
              v = uok ? v : 0;
              acc[t] = fmaf((float)v, FMT == KT_FMT_TERN ? __uint_as_float(sa[0][j][t]) * d : d * __uint_as_float(sa[0][j][t]), acc[t]);
              if(DBG && uok && row < R) dbg[((long long)(p0 + t0 + t) * R + row) * NU + u] = v;
            }
          }
        }
      }
      kt_wave_sync();                                                /* the staging is rewritten next */
    }
    KT_GTS(2);
    float y[MT];
#pragma unroll
    for(int t = 0; t < MT; ++t) y[t] = kt_row_sum(acc[t]);
    if(c == 0){
#pragma unroll
      for(int t = 0; t < MT; ++t) red[(ks * MT + t) * 8 + r] = y[t];
    }
    __syncthreads();                                                 /* every wave runs the same token chunks */
    if(ks == 0 && c == 0){
      float vv[MT];
#pragma unroll
      for(int t = 0; t < MT; ++t){
        float v = red[t * 8 + r];
        for(int k = 1; k < KS; ++k) v += red[(k * MT + t) * 8 + r];
        vv[t] = v;
      }
#pragma unroll
      for(int t = 0; t < MT; ++t){
        if(!GRP && a.hp){                                             /* rows 2t, 2t + 1 -> token t (MT even) */
          if(MT > 1 && !(t & 1) && t < nt && row < R) yout[(long long)((t0 + t) >> 1) * ldy + row] = vv[t] + vv[t + 1 < MT ? t + 1 : t];
        } else if(t < nt && row < R){
          yout[(long long)(p0 + t0 + t) * ldy + row] = vv[t];
        }
      }
    }
    __syncthreads();
  }
  KT_GTS(3);
}

/* one token of a dense ternary launch whose slices have at most KT_SL steps (the one-token decode): the body above
   for M = 1 with the loads in another order. The activation rows of the slice's steps go out first, then the
   weights (the first halves c0 of every step, then the c1 halves, then the scales): loads retire in order, so the
   staging waits for the activations alone while the weights are still in flight, and each step's first half can be
   taken before the last weight bytes land. The same chains, butterfly and slice order, so the same bits. */
template <bool DBG>
__device__ __forceinline__ void kt_gemv_one_body(const KtGemvArgs& a, const int8_t* __restrict__ xq,
                                                 const float* __restrict__ xs, const int* __restrict__ xa,
                                                 int32_t* __restrict__ dbg, int KS){
  extern __shared__ __attribute__((aligned(16))) uint8_t kt_lds[];
  using F = KtFlat<KT_FMT_TERN, 1>;
  constexpr int UW = F::UW, UP = F::UP, SL = KT_SL;
  const int NU = a.NU, S = kt_steps(NU);
  const int lane = threadIdx.x & 63, ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), r = lane & 7, c = lane >> 3;
  const int g = blockIdx.x;
  int mi = 0;
  if(a.nmat > 1 && g >= a.mat[1].rg0) mi = 1;
  if(a.nmat > 2 && g >= a.mat[2].rg0) mi = 2;
  const KtMat& m = a.mat[mi];
  const uint4* __restrict__ wb = (const uint4*)m.codes;
  const uint16_t* __restrict__ sb = m.scales;
  const int R = m.R, rg = g - m.rg0, row = rg * KT_RG + r;
  const int s_lo = ks * S / KS, ns = (ks + 1) * S / KS - s_lo;      /* this slice's steps (1 .. SL) */
  uint8_t* xw = kt_lds + (size_t)ks * F::XW;                         /* [SL][8][UP] */
  float* red = (float*)(kt_lds + (size_t)KS * F::XW);                /* [KS][8] */
  /* the activation rows of the slice's steps, the lane's unit scales and sums */
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
  /* every weight offset (an integer select: a unit past the slice or the matrix reads offset 0), then the loads */
  unsigned o0[SL], o1[SL], os[SL];
#pragma unroll
  for(int j = 0; j < SL; ++j){
    const int s = s_lo + j, u = s * KT_KL + c;
    const bool ok = j < ns && u < NU;
    o0[j] = ok ? (unsigned)kt_widx(NU, rg, s, 0, c, r) : 0u;
    o1[j] = ok ? (unsigned)kt_widx(NU, rg, s, 1, c, r) : 0u;
    os[j] = ok ? (unsigned)kt_sidx(NU, rg, u, r) : 0u;
  }
  KtStep w[SL];
#pragma unroll
  for(int j = 0; j < SL; ++j) w[j].c0 = kt_ldnt(wb + o0[j]);
#pragma unroll
  for(int j = 0; j < SL; ++j) w[j].c1 = kt_ldnt(wb + o1[j]);
#pragma unroll
  for(int j = 0; j < SL; ++j) w[j].hs = sb[os[j]];
  __builtin_amdgcn_sched_barrier(0);
  kt_pin<SL>(&stg[0], &sa[0][0]);                                    /* every load above is issued before a write */
  {
    const bool in = o < KT_KL * UW;
    const int lo = (o / UW) * UP + o % UW;
#pragma unroll
    for(int j = 0; j < SL; ++j) *(uint4*)(xw + (in ? j * KT_KL * UP + lo : F::XW - 16)) = stg[j];
  }
  kt_wave_sync();
  float acc = 0.0f;
#pragma unroll
  for(int j = 0; j < SL; ++j){
    const int u = (s_lo + j) * KT_KL + c;
    if(j < ns){                                                      /* wave-uniform */
      const bool uok = u < NU;
      const float d = uok ? kt_h2f(w[j].hs) : 0.0f;
      int v = kt_unit_lds<KT_FMT_TERN>(w[j].c0, w[j].c1, xw + (j * KT_KL + (uok ? c : 0)) * UP) - (int)sa[1][j];
      v = uok ? v : 0;
      acc = fmaf((float)v, __uint_as_float(sa[0][j]) * d, acc);
      if(DBG && uok && row < R) dbg[(long long)row * NU + u] = v;
    }
  }
  const float y = kt_row_sum(acc);
  if(c == 0) red[ks * 8 + r] = y;
  __syncthreads();
  if(ks == 0 && c == 0){
    float v = red[r];
    for(int k = 1; k < KS; ++k) v += red[k * 8 + r];
    if(row < R) m.y[row] = v;
  }
}

/* one token a chunk: held to 64 VGPRs (8 waves a SIMD), so three 9-wave blocks fit a CU and the widest products
   run in one round of blocks */
template <int FMT, int MT, bool DBG, bool GRP>
__global__ void __launch_bounds__(64 * KT_KSMAX) __attribute__((amdgpu_waves_per_eu(8)))
k_gemv_flat1(const KtGemvArgs a, const KtGroupedArgs ga, const int8_t* __restrict__ xq, const float* __restrict__ xs,
             const int* __restrict__ xa, int32_t* __restrict__ dbg, int KS){
  if constexpr(KT_FLAT1_ONE && FMT == KT_FMT_TERN && MT == 1 && !GRP){
    /* one token with slices of at most KT_SL steps (uniform): activations first */
    if(a.M == 1 && !a.hp && kt_steps(a.NU) <= KT_SL * KS){ kt_gemv_one_body<DBG>(a, xq, xs, xa, dbg, KS); return; }
  }
  kt_gemv_flat_body<FMT, MT, DBG, GRP>(a, ga, xq, xs, xa, dbg, KS);
}
template <int FMT, int MT, bool DBG, bool GRP>
__global__ void __launch_bounds__(64 * KT_KSMAX)
k_gemv_flat(const KtGemvArgs a, const KtGroupedArgs ga, const int8_t* __restrict__ xq, const float* __restrict__ xs,
            const int* __restrict__ xa, int32_t* __restrict__ dbg, int KS){
  kt_gemv_flat_body<FMT, MT, DBG, GRP>(a, ga, xq, xs, xa, dbg, KS);
}
