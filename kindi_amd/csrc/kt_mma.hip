/* kt_mma.hip - the decode product on the matrix cores for up to 32 tokens (passes of 16; the launcher takes it from 3
   tokens) (k_tc_mv*, tc_hip.cu:180-240, at the verify widths spec.py:45 takes them): ternary
   weights (kt2) against int8 token rows, the same numbers and the
   same summation tree as k_gemv_flat, so a token's bits do not depend on which of the two kernels ran it.

   Block: KS waves over one tile of 32 weight rows (4 row groups of one matrix); wave ks takes the K slice ks (steps
   [ks S / KS, (ks + 1) S / KS), at most 2); grid.y the passes of 16 tokens. A unit (128 columns) is 4
   V_MFMA_I32_32X32X32_I8 (token rows 16 .. 31 of the A operand are zero): lane l holds weight row l % 32 (B operand)
   and token l % 32 (A operand), both for the columns 64 h + 16 i .. + 15 of the unit in
   MFMA i (h = l / 32), so the 4 MFMAs cover the unit's 128 columns once each and give its exact int32 value
   v(t, r) (any pairing of columns gives the same integer). A lane's kt2 load is exactly its row's 64 columns of
   the unit (kt_widx with half h), unpacked to signed trits (shift, mask, v_perm byte lookup); its activations are
   the same 64 columns of its token, read from L2 (tokens past the pass or M are zero and not loaded).

   The fp32 epilogue takes k_gemv_flat's order: for each k-lane c (0..7) of the step layout, the chain over the
   slice's units 8 s + c in increasing s, fmaf((float)v, XS[t][u] * d[r][u], .); then ((c0 + c1) + (c2 + c3)) +
   ((c4 + c5) + (c6 + c7)) (the xor butterfly's result) in registers; then the slices in order, in LDS. D register
   layout (32x32x32 i8 on gfx950): lane l register e holds column l % 32 (the weight row) and row (e % 4) + 8 (e / 4)
   + 4 (l / 32) (the token). */
#include "kt_gemv.h"

typedef int kt_v4i __attribute__((ext_vector_type(4)));
typedef int kt_v16i __attribute__((ext_vector_type(16)));

#define KM_ROWS 32                    /* weight rows a tile */
#define KM_TOK 16                     /* tokens a pass */


/* 4 digits (0/1/2, one per byte) -> 4 signed trits (-1/0/+1): byte lookup in 0x000100FF */
__device__ __forceinline__ int km_trits(uint32_t dig){ return (int)__builtin_amdgcn_perm(0x000100FFu, 0x000100FFu, dig); }

/* the token of D register e of lane l */
__device__ __forceinline__ int km_tok(int e, int lane){ return (e & 3) + 8 * (e >> 2) + 4 * (lane >> 5); }

template <int NT, bool DBG, int LB>   /* NT: the token rows of a pass (16: D registers e < 8); LB: threads a block */
__global__ void __launch_bounds__(LB) k_gemv_mma(const KtGemvArgs a, const int8_t* __restrict__ xq,
                                                            const float* __restrict__ xs,
                                                            int32_t* __restrict__ dbg, int KS){
  constexpr int NE = NT / 2;                                     /* D registers that hold used tokens */
  constexpr int KM_PF = LB <= 256 ? 4 : LB <= 640 ? 2 : 0;        /* activation units loaded ahead (register room) */
  extern __shared__ __attribute__((aligned(16))) uint8_t kt_lds[];
  float* red = (float*)kt_lds;                                   /* [KS][NT][32] slice sums */
  const int NU = a.NU, S = kt_steps(NU);
  const int lane = threadIdx.x & 63, ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = lane >> 5, lr = lane & 31;
  const int tile = blockIdx.x, t0 = blockIdx.y * KM_TOK;
  KT_GTS(0);
  int mi = 0;
  if(a.nmat > 1 && tile >= a.mat[1].pad) mi = 1;
  if(a.nmat > 2 && tile >= a.mat[2].pad) mi = 2;
  const KtMat& m = a.mat[mi];
  const int rg = (tile - m.pad) * 4 + (lr >> 3), r = lr & 7, row = rg * KT_RG + r;
  const bool rok = row < m.R;
  const int nt = min(KM_TOK, a.M - t0);
  const int tok = t0 + lr;                                        /* this lane's A row (token) */
  const bool tok_ok = lr < nt;
  const int s_lo = ks * S / KS, ns = (ks + 1) * S / KS - s_lo;   /* this slice's steps (1 or 2) */
  const uint4* __restrict__ wb = (const uint4*)m.codes;
  const uint16_t* __restrict__ sb = m.scales;

  /* the slice's XS [16 units][16 tokens] (clamped, unconditional loads) first: they go to this wave's LDS region
     after the weight and the first activation loads are issued, so that wait leaves those in flight (loads retire
     in order); the epilogue reads them from LDS, and every global load below is unconditional, so the compiler's
     wait counts stay exact and the activation loads of later units run ahead */
  float* xsl = (float*)(kt_lds + (size_t)KS * NT * 32 * 4) + (size_t)ks * 256;
  float xsv[4];
#pragma unroll
  for(int q = 0; q < 4; ++q){
    const int idx = lane + 64 * q, n = idx >> 4, tl = idx & 15;
    const int u = (s_lo + (n >> 3)) * KT_KL + (n & 7);
    const int t = t0 + tl < a.M ? t0 + tl : t0;
    xsv[q] = xs[(long long)t * a.ldxs + (u < NU ? u : 0)];
  }

  float part[NE];                                                  /* the combined chains of this slice */
  float t01[NE], t23[NE], t45[NE], pend[NE];
#pragma unroll
  for(int e = 0; e < NE; ++e){ part[e] = 0.0f; t01[e] = 0.0f; t23[e] = 0.0f; t45[e] = 0.0f; pend[e] = 0.0f; }

  /* the slice's 16 units in k-lane-major order (c, then the two steps), fully unrolled with unconditional loads
     (a unit past the slice or the matrix reads offset 0 and a zero token), so loads run ahead of their products */
  uint4 wq[2][KT_KL];
  uint16_t hq[2][KT_KL];
#pragma unroll
  for(int c = 0; c < KT_KL; ++c)
#pragma unroll
    for(int j = 0; j < 2; ++j){
      const int s = s_lo + j, u = s * KT_KL + c;
      const bool ok = rok && j < ns && u < NU;
      wq[j][c] = kt_ldnt(wb + (ok ? kt_widx(NU, rg, s, h, c, r) : 0));
      hq[j][c] = sb[ok ? kt_sidx(NU, rg, u, r) : 0];
    }
  /* a buffer resource over the M token rows: lanes past the pass's tokens read from offset 2^30, beyond the range
     (the launcher keeps M ldq below it), which returns zeros without a memory access */
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)xq, (short)0, a.M * a.ldq, 0x00020000);
  const uint32_t xoff = tok_ok ? (uint32_t)(tok * a.ldq + 64 * h) : (1u << 30);
  uint4 xa[KM_PF > 0 ? KM_PF : 1][4];
  auto ld_act = [&](int n, uint4* dst){
    const int c = n >> 1, j = n & 1, u = (s_lo + j) * KT_KL + c;
    const int uu = (j < ns && u < NU) ? u : 0;
#pragma unroll
    for(int i = 0; i < 4; ++i)
      dst[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, xoff + uu * 128 + 16 * i, 0, 0));
  };
#pragma unroll
  for(int n = 0; n < KM_PF; ++n) ld_act(n, xa[n]);
#pragma unroll
  for(int q = 0; q < 4; ++q) xsl[lane + 64 * q] = xsv[q];
  kt_wave_sync();
  KT_GTS(1);
#pragma unroll
  for(int c = 0; c < KT_KL; ++c){
    float chain[NE];
#pragma unroll
    for(int e = 0; e < NE; ++e) chain[e] = 0.0f;
#pragma unroll
    for(int j = 0; j < 2; ++j){
      const int n = 2 * c + j, s = s_lo + j, u = s * KT_KL + c;
      const bool uok = j < ns && u < NU;                        /* wave-uniform */
      uint4 xa4[4];
      if constexpr(KM_PF == 0) ld_act(n, xa4);
      else {
#pragma unroll
        for(int i = 0; i < 4; ++i) xa4[i] = xa[n % KM_PF][i];
        if(n + KM_PF < 2 * KT_KL) ld_act(n + KM_PF, xa[n % KM_PF]);
      }
      if(uok){
        const uint32_t ww[4] = {wq[j][c].x, wq[j][c].y, wq[j][c].z, wq[j][c].w};
        const float d = rok ? kt_h2f(hq[j][c]) : 0.0f;
        kt_v16i acc;
#pragma unroll
        for(int e = 0; e < 16; ++e) acc[e] = 0;
#pragma unroll
        for(int i = 0; i < 4; ++i){
          kt_v4i B, A;
          B[0] = km_trits(ww[i] & 0x03030303u);
          B[1] = km_trits((ww[i] >> 2) & 0x03030303u);
          B[2] = km_trits((ww[i] >> 4) & 0x03030303u);
          B[3] = km_trits((ww[i] >> 6) & 0x03030303u);
          A[0] = (int)xa4[i].x; A[1] = (int)xa4[i].y; A[2] = (int)xa4[i].z; A[3] = (int)xa4[i].w;
          acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, acc, 0, 0, 0);
        }
        /* epilogue: the k-lane chain, fmaf((float)v, XS * d, .) */
#pragma unroll
        for(int e = 0; e < NE; ++e){
          const int t = t0 + km_tok(e, lane);
          const float sx = xsl[(j * 8 + c) * 16 + km_tok(e, lane)];
          chain[e] = fmaf((float)acc[e], sx * d, chain[e]);
          if(DBG && t < a.M && rok) dbg[((long long)t * m.R + row) * NU + u] = acc[e];
        }
      }
    }
    /* the butterfly's tree over c, as it completes */
#pragma unroll
    for(int e = 0; e < NE; ++e){
      if(c == 0 || c == 2 || c == 4 || c == 6) pend[e] = chain[e];
      else if(c == 1) t01[e] = pend[e] + chain[e];
      else if(c == 3) t23[e] = t01[e] + (pend[e] + chain[e]);          /* (c0 + c1) + (c2 + c3) */
      else if(c == 5) t45[e] = pend[e] + chain[e];
      else part[e] = t23[e] + (t45[e] + (pend[e] + chain[e]));          /* ... + ((c4 + c5) + (c6 + c7)) */
    }
  }
  /* slices in order */
  KT_GTS(2);
#pragma unroll
  for(int e = 0; e < NE; ++e) red[((size_t)ks * NT + km_tok(e, lane)) * 32 + lr] = part[e];
  __syncthreads();
  if(ks == 0){
    /* slices outer, tokens inner: each pass's 8 LDS reads are issued together (a token's sum keeps slice order) */
    float v[NE];
#pragma unroll
    for(int e = 0; e < NE; ++e) v[e] = red[(size_t)km_tok(e, lane) * 32 + lr];
    for(int k = 1; k < KS; ++k){
      float w[NE];
#pragma unroll
      for(int e = 0; e < NE; ++e) w[e] = red[((size_t)k * NT + km_tok(e, lane)) * 32 + lr];
#pragma unroll
      for(int e = 0; e < NE; ++e) v[e] += w[e];
    }
#pragma unroll
    for(int e = 0; e < NE; ++e){
      const int t = t0 + km_tok(e, lane);                        /* even e: an even row, its pair in e + 1 */
      if(a.hp){
        if(!(e & 1) && t < a.M && rok) m.y[(long long)(t >> 1) * m.ldy + row] = v[e] + v[e + 1];
      } else if(t < a.M && rok) m.y[(long long)t * m.ldy + row] = v[e];
    }
  }
  KT_GTS(3);
}

template __global__ void k_gemv_mma<16, false, 64 * KT_KSMAX>(const KtGemvArgs, const int8_t*, const float*, int32_t*, int);
template __global__ void k_gemv_mma<16, true, 64 * KT_KSMAX>(const KtGemvArgs, const int8_t*, const float*, int32_t*, int);

/* ------------------------------------------------------------------ ternary, 16 tokens, V_MFMA_I32_16X16X64_I8
   k_gemv_m16: the numbers, tree and block shape of k_gemv_mma (a tile of 32 weight rows, wave ks = K slice ks,
   grid.y = passes of 16 tokens) on 16x16x64 MFMAs, which have no idle token rows at 16 tokens and give each unit two
   independent accumulator chains:
   - lane l = 16 g + n loads one 16-byte kt2 chunk of the unit: half g % 2 (columns 64 (g % 2) .. + 63) of row
     16 (g / 2) + n of the tile, so the wave's 64 loads are the unit's 1 KB in contiguous 128-byte runs;
   - a 4 x 4 transpose of words across the four 16-lane rows (two permlane32 swaps, two permlane16 swaps) leaves lane
     (g, n) with word g of the four chunks of its row n: for chunk m (row block m / 2, half m % 2) the four lanes of
     row n hold its 64 columns 64 (m % 2) + 16 g .. + 15 (g = 0 .. 3); as unsigned digits (0 / 1 / 2, one a byte)
     they are the B operand (column n = the weight row), and the A operand is token n's activations of the same
     columns (V_MFMA_I32_16X16X64_I8: lane 16 g + n holds row / column n, k = 16 g .. + 15 in byte order, measured);
   - row block b chains its two halves on one accumulator: lane (g, n) register j = sum d q (token 4 g + j, row
     16 b + n); minus XA (sum q) it is the exact int32 unit value sum t q (any pairing of columns gives the same
     integer).
   The fp32 epilogue is k_gemv_mma's (and k_gemv_flat's) order: per k-lane c the chain over the slice's units 8 s + c
   in increasing s, fmaf((float)v, XS[t][u] * d[r][u], .), the butterfly's tree over c, the slices in order. */
__device__ __forceinline__ void km_swap32(unsigned& a, unsigned& b){
  const auto t = __builtin_amdgcn_permlane32_swap(a, b, false, false); a = t[0]; b = t[1];
}
__device__ __forceinline__ void km_swap16(unsigned& a, unsigned& b){
  const auto t = __builtin_amdgcn_permlane16_swap(a, b, false, false); a = t[0]; b = t[1];
}
/* one kt2 word -> its 16 digits d = t + 1 (0 / 1 / 2) in column order, as unsigned bytes */
__device__ __forceinline__ kt_v4i km_digits16(uint32_t w){
  kt_v4i B;
  B[0] = (int)(w & 0x03030303u);
  B[1] = (int)((w >> 2) & 0x03030303u);
  B[2] = (int)((w >> 4) & 0x03030303u);
  B[3] = (int)((w >> 6) & 0x03030303u);
  return B;
}

/* up to 10 K slices, activations 2 units ahead. The B operands are the unsigned digits d = t + 1 (masks and shifts
   of the kt2 word, no lookup): an MFMA then gives the exact integer sum d q, and the unit value is v = sum d q - XA
   (XA = sum q, the quantizer's), the same integer as sum t q. The weights, scales, XS and XA are read through buffer
   resources that span exactly their buffers, with 32-bit offsets.
   KQ = 1: wave ks takes the whole slice ks (640 threads, 3 waves a SIMD).
   KQ = 4: each slice's k-lanes are split over 4 waves, wave (sg, q) taking k-lanes 2 q and 2 q + 1 of slices sg,
   sg + G, ... (MS: G = 4 slice groups for launches of more than 4 slices, so a block has at most 16 waves; else
   G = KS, one slice a wave), staging only those units' XS and XA. For each of its slices a wave writes the pair sum
   p_q = chain(2 q) + chain(2 q + 1) to LDS, and wave 0 forms the butterfly's tree (p0 + p1) + (p2 + p3), which is
   the KQ = 1 tree ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7)), then the slices in order: the same bits with 4
   times the waves. KQ = 2 (with MS, G = 8): k-lane quads, a wave's sum (c0 + c1) + (c2 + c3) of its four and wave 0
   adding the two quads. */
#ifdef KT_TRACE
#define KT_M16TS(k) do { if(kt_trace_on && lane == 0 && blockIdx.x < 512 && blockIdx.y == 0) \
    kt_trace_buf[(blockIdx.x * 16 + wvi) * 8 + (k)] = __builtin_amdgcn_s_memrealtime(); } while(0)
#else
#define KT_M16TS(k) do {} while(0)
#endif
template <bool DBG, int KQ, bool MS>
__global__ void __launch_bounds__(KQ == 1 ? 640 : 1024) k_gemv_m16(const KtGemvArgs a, const int8_t* __restrict__ xq,
                                                  const float* __restrict__ xs, const int* __restrict__ xav,
                                                  int32_t* __restrict__ dbg, int KS){
  /* activation units loaded ahead: 2 (measured on MI355X, 27B-class step at 16 tokens: 1, 2, 3, 4, 6 units ahead
     4.03, 3.85, 3.87, 3.92, 4.03 ms; even at 3 - 8 tokens) */
  constexpr int NT = KM_TOK, KM_PF = 2;                          /* tokens a pass */
  constexpr int CW = KT_KL / KQ;                                 /* k-lanes a wave */
  extern __shared__ __attribute__((aligned(16))) uint8_t kt_lds[];
  float* red = (float*)kt_lds;                                   /* [KS][KQ][2][64] float4: the slice (pair) sums */
  const int NU = a.NU, S = kt_steps(NU);
  const int lane = threadIdx.x & 63, wvi = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  /* KQ = 1: wave ks = slice ks. KQ = 4: G slice groups, wave (sg, q) takes k-lanes 2 q, 2 q + 1 of slices sg,
     sg + G, sg + 2 G, ... */
  const int G = MS ? 16 / KQ : KS;                               /* MS: more slices than groups */
  const int sg = wvi / KQ, q = wvi % KQ, cb = q * CW;            /* slice group, quarter, first k-lane */
  const int g = lane >> 4, n = lane & 15;
  const int tile = blockIdx.x, t0 = blockIdx.y * NT;
  KT_M16TS(0);
  int mi = 0;
  if(a.nmat > 1 && tile >= a.mat[1].pad) mi = 1;
  if(a.nmat > 2 && tile >= a.mat[2].pad) mi = 2;
  const KtMat& m = a.mat[mi];
  const int rg0 = (tile - m.pad) * 4;                            /* the tile's first row group (of the matrix) */
  const int crg = rg0 + 2 * (g >> 1) + (n >> 3), cr = n & 7, ch = g & 1;   /* this lane's chunks */
  const bool cok = crg * KT_RG + cr < m.R;
  /* the rows of this lane's results: 16 b + n of the tile (row block b = 0, 1) */
  int orow[2];
  bool ook[2];
#pragma unroll
  for(int b = 0; b < 2; ++b){ orow[b] = (rg0 + 2 * b + (n >> 3)) * KT_RG + cr; ook[b] = orow[b] < m.R; }
  const int nt = min(NT, a.M - t0);
  const int nrg = kt_r8(m.R);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc((void*)m.codes, (short)0, nrg * NU * 256, 0x00020000);
  const __amdgpu_buffer_rsrc_t hr = __builtin_amdgcn_make_buffer_rsrc((void*)m.scales, (short)0, nrg * NU * 16, 0x00020000);
  const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc((void*)xs, (short)0, a.M * a.ldxs * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc((void*)xav, (short)0, a.M * a.ldxs * 4, 0x00020000);

  /* the units' XS and XA [16 units][16 tokens] to this wave's LDS region (after the weight loads are issued) */
  float* xsl = (float*)(kt_lds + (size_t)KS * KQ * NT * 32 * 4) + (size_t)wvi * 512;
  int* xal = (int*)(xsl + 256);
  /* activations through a buffer resource over the M token rows (lanes past the pass's tokens: past the range,
     zeros without a memory access) */
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)xq, (short)0, a.M * a.ldq, 0x00020000);
  const uint32_t xoff = n < nt ? (uint32_t)((t0 + n) * a.ldq + 16 * g) : (1u << 30);
  for(int it = 0, ks = sg; MS ? ks < KS : it < 1; ++it, ks += G){                /* !MS: one slice a wave */
  const int s_lo = ks * S / KS, ns = (ks + 1) * S / KS - s_lo;   /* this slice's steps (1 or 2) */
  /* entry (j 8 + c) 16 + token of the region: KQ = 1 stages the slice's 16 units, KQ = 4 only its own 4 (k-lanes cb,
     cb + 1 of both steps) */
  constexpr int NI = 4 / KQ;
  float xsv[NI];
  int xav4[NI];
  int xdst[NI];
#pragma unroll
  for(int i = 0; i < NI; ++i){
    const int idx = lane + 64 * i, un = idx >> 4, tl = idx & 15;
    const int j = un / CW, c = cb + un % CW;                     /* the wave's units: CW k-lanes, 2 steps */
    const int u = (s_lo + j) * KT_KL + c;
    const int t = t0 + tl < a.M ? t0 + tl : t0;
    const uint32_t o = (uint32_t)(t * a.ldxs + (u < NU ? u : 0)) * 4;
    xsv[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sr, o, 0, 0));
    xav4[i] = (int)__builtin_amdgcn_raw_buffer_load_b32(ar, o, 0, 0);
    xdst[i] = (j * 8 + c) * 16 + tl;
  }
  float part[8], t01[8], t23[8], t45[8], pend[8];
#pragma unroll
  for(int e = 0; e < 8; ++e){ part[e] = 0.0f; t01[e] = 0.0f; t23[e] = 0.0f; t45[e] = 0.0f; pend[e] = 0.0f; }

  uint4 xa[KM_PF][2];
  auto ld_act = [&](int un, uint4* dst){                         /* the wave's unit un = 2 (c - cb) + j: both halves */
    const int c = cb + (un >> 1), j = un & 1, u = (s_lo + j) * KT_KL + c;
    const int uu = (j < ns && u < NU) ? u : 0;
    dst[0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, xoff + uu * 128, 0, 0));
    dst[1] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, xoff + uu * 128 + 64, 0, 0));
  };
  /* the first units' activations before the weights: loads retire in order, so unit 0 can start as soon as its own
     weights have landed rather than after the whole slice */
#pragma unroll
  for(int un = 0; un < KM_PF; ++un) ld_act(un, xa[un]);
  /* the slice's 16 units' chunks (k-lane-major) and both row blocks' scales (b = 0 | b = 1 << 16), unconditional */
  uint4 wq[2][CW];
  uint32_t hq[2][CW];
#pragma unroll
  for(int cc = 0; cc < CW; ++cc)
#pragma unroll
    for(int j = 0; j < 2; ++j){
      const int c = cb + cc, s = s_lo + j, u = s * KT_KL + c;
      const bool ok = j < ns && u < NU;
      const uint32_t wo = ok && cok ? (uint32_t)kt_widx(NU, crg, s, ch, c, cr) * 16 : 0u;
      wq[j][cc] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, wo, 0, 2));
      /* rows past R read past the resource: a zero scale, so their chains stay zero without a select */
      const uint32_t h0 = __builtin_amdgcn_raw_buffer_load_b16(
          hr, ok && ook[0] ? (uint32_t)kt_sidx(NU, rg0 + (n >> 3), u, cr) * 2 : (1u << 31), 0, 0);
      const uint32_t h1 = __builtin_amdgcn_raw_buffer_load_b16(
          hr, ok && ook[1] ? (uint32_t)kt_sidx(NU, rg0 + 2 + (n >> 3), u, cr) * 2 : (1u << 31), 0, 0);
      hq[j][cc] = h0 | h1 << 16;
    }
#pragma unroll
  for(int i = 0; i < NI; ++i){ xsl[xdst[i]] = xsv[i]; xal[xdst[i]] = -xav4[i]; }        /* XA negated */
  kt_wave_sync();
  KT_M16TS(1);
#pragma unroll
  for(int cc = 0; cc < CW; ++cc){
    const int c = cb + cc;
    float chain[8];                                              /* element 4 b + e: row block b, token 4 g + e */
#pragma unroll
    for(int e = 0; e < 8; ++e) chain[e] = 0.0f;
#pragma unroll
    for(int j = 0; j < 2; ++j){
      const int un = 2 * cc + j, u = (s_lo + j) * KT_KL + c;
      const bool uok = j < ns && u < NU;                         /* wave-uniform */
      const uint4 x0 = xa[un % KM_PF][0], x1 = xa[un % KM_PF][1];
      if(un + KM_PF < 2 * CW) ld_act(un + KM_PF, xa[un % KM_PF]);
      if(uok){
        /* word g of the four chunks of row n */
        unsigned w0 = wq[j][cc].x, w1 = wq[j][cc].y, w2 = wq[j][cc].z, w3 = wq[j][cc].w;
        km_swap32(w0, w2); km_swap32(w1, w3);
        km_swap16(w0, w1); km_swap16(w2, w3);
        const kt_v4i A0 = {(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w};
        const kt_v4i A1 = {(int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
        /* both chains start from -XA of tokens 4 g .. + 3 (staged negated), so they end at v = sum d q - XA */
        const int4 xa4 = *(const int4*)(xal + (j * 8 + c) * 16 + 4 * g);
        const kt_v4i cx = {xa4.x, xa4.y, xa4.z, xa4.w};
        kt_v4i d0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, km_digits16(w0), cx, 0, 0, 0);   /* row block 0, half 0 */
        kt_v4i d1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, km_digits16(w2), cx, 0, 0, 0);   /* row block 1, half 0 */
        d0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, km_digits16(w1), d0, 0, 0, 0);          /* row block 0, half 1 */
        d1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, km_digits16(w3), d1, 0, 0, 0);          /* row block 1, half 1 */
        const float dd0 = kt_h2f((uint16_t)hq[j][cc]), dd1 = kt_h2f((uint16_t)(hq[j][cc] >> 16));
        const float4 sx = *(const float4*)(xsl + (j * 8 + c) * 16 + 4 * g);                /* tokens 4 g .. + 3 */
        const float sxv[4] = {sx.x, sx.y, sx.z, sx.w};
#pragma unroll
        for(int e = 0; e < 4; ++e){
          chain[e] = fmaf((float)d0[e], sxv[e] * dd0, chain[e]);
          chain[4 + e] = fmaf((float)d1[e], sxv[e] * dd1, chain[4 + e]);
          if(DBG){
            const int t = t0 + 4 * g + e;
            if(t < a.M && ook[0]) dbg[((long long)t * m.R + orow[0]) * NU + u] = d0[e];
            if(t < a.M && ook[1]) dbg[((long long)t * m.R + orow[1]) * NU + u] = d1[e];
          }
        }
      }
    }
    /* the butterfly's tree over c, as it completes (KQ = 4: this wave's pair sum) */
#pragma unroll
    for(int e = 0; e < 8; ++e){
      if constexpr(KQ == 1){
        if(c == 0 || c == 2 || c == 4 || c == 6) pend[e] = chain[e];
        else if(c == 1) t01[e] = pend[e] + chain[e];
        else if(c == 3) t23[e] = t01[e] + (pend[e] + chain[e]);
        else if(c == 5) t45[e] = pend[e] + chain[e];
        else part[e] = t23[e] + (t45[e] + (pend[e] + chain[e]));
      } else if constexpr(KQ == 2){                              /* (c0 + c1) + (c2 + c3) of the wave's four */
        if(cc == 0 || cc == 2) pend[e] = chain[e];
        else if(cc == 1) t01[e] = pend[e] + chain[e];
        else part[e] = t01[e] + (pend[e] + chain[e]);
      } else {
        if(cc == 0) pend[e] = chain[e];
        else part[e] = pend[e] + chain[e];
      }
    }
  }
  KT_M16TS(2);
  /* slices in order (KQ = 4: the pair sums of a slice first, (p0 + p1) + (p2 + p3)) */
  /* a lane's 8 sums as two float4 at [slice][quarter][half][lane]: 16-byte LDS accesses, conflict free */
  {
    float4* r4 = (float4*)red + (size_t)(ks * KQ + q) * 128 + lane;
    r4[0] = make_float4(part[0], part[1], part[2], part[3]);
    r4[64] = make_float4(part[4], part[5], part[6], part[7]);
  }
  }                                                              /* the wave's slices */
  __syncthreads();
  KT_M16TS(3);
  if(wvi == 0){
    auto slice = [&](int k, float (&w)[8]){
      float p[KQ][8];
#pragma unroll
      for(int qq = 0; qq < KQ; ++qq){
        const float4* r4 = (const float4*)red + (size_t)(k * KQ + qq) * 128 + lane;
        const float4 lo = r4[0], hi = r4[64];
        p[qq][0] = lo.x; p[qq][1] = lo.y; p[qq][2] = lo.z; p[qq][3] = lo.w;
        p[qq][4] = hi.x; p[qq][5] = hi.y; p[qq][6] = hi.z; p[qq][7] = hi.w;
      }
#pragma unroll
      for(int e = 0; e < 8; ++e){
        if constexpr(KQ == 1) w[e] = p[0][e];
        else if constexpr(KQ == 2) w[e] = p[0][e] + p[1][e];
        else w[e] = (p[0][e] + p[1][e]) + (p[2][e] + p[3][e]);
      }
    };
    float v[8];
    slice(0, v);
    for(int k = 1; k < KS; ++k){
      float w[8];
      slice(k, w);
#pragma unroll
      for(int e = 0; e < 8; ++e) v[e] += w[e];
    }
#pragma unroll
    for(int e = 0; e < 8; ++e){
      const int t = t0 + 4 * g + (e & 3);                        /* even e: an even row, its pair in e + 1 */
      if(a.hp){
        if(!(e & 1) && t < a.M && ook[e >> 2]) m.y[(long long)(t >> 1) * m.ldy + orow[e >> 2]] = v[e] + v[e + 1];
      } else if(t < a.M && ook[e >> 2]) m.y[(long long)t * m.ldy + orow[e >> 2]] = v[e];
    }
    KT_M16TS(4);
  }
}

#define KM16_INST(DBG, KQ, MS) template __global__ void k_gemv_m16<DBG, KQ, MS>(const KtGemvArgs, const int8_t*, \
    const float*, const int*, int32_t*, int);
KM16_INST(false, 1, false) KM16_INST(true, 1, false) KM16_INST(false, 4, false) KM16_INST(true, 4, false)
KM16_INST(false, 4, true) KM16_INST(true, 4, true) KM16_INST(false, 2, true) KM16_INST(true, 2, true)
#undef KM16_INST

/* ------------------------------------------------------------------ q8_0 on the matrix cores
   The q8_0 product (kq8 weights against int8 rows with per-32 scales, lt_mv_q8 lightning.cu:258-284, k_q8
   dsv41_gpu.cu:131-296) with the same numbers and tree as k_gemv_flat's q8_0 mode, dense (one matrix, tokens 0 ..
   M - 1) or grouped (GRP: one active expert a block row, its token list: entry p reads input row xrow[p] or p and
   writes output row p, lt_mm_* lightning.cu:958-1168). A q8_0 unit (32 columns) is one V_MFMA_I32_32X32X32_I8:
   lane l holds weight row l % 32 and token l % 32, columns 16 h .. 16 h + 15 of the unit (h = l / 32), which is
   exactly one 16-byte load of the kq8 layout (kt_widx with half h). Block: one tile of 32 weight rows (4 row
   groups); with KS waves, wave ks takes K slice ks and its weights are loaded once for every pass of 16 tokens of
   the block's list; with MS, W waves take the slices in turn (wave w: slices w, w + W, ...), reading each slice's
   weights again every pass. Epilogue as k_gemv_flat: per k-lane c the chain fmaf((float)v, d * D[t][u], .) over the slice's
   units 8 s + c, the butterfly's tree over c, the slices in order. */
#define KM_Q8_KS 8                    /* at most 8 K slices (q8_0 C <= 4096): 256 VGPRs a lane */
template <bool GRP, bool DBG, bool MS>   /* MS: wave w takes slices w, w + W, ... (W waves a block) */
__global__ void __launch_bounds__(64 * KM_Q8_KS) k_q8_mma(const KtGemvArgs a, const KtGroupedArgs ga,
                                                          const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                          int32_t* __restrict__ dbg, int KS){
  constexpr int NT = KM_TOK, NE = NT / 2;
  extern __shared__ __attribute__((aligned(16))) uint8_t kt_lds[];
  float* red = (float*)kt_lds;                                   /* [KS][NT][32] slice sums */
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = blockDim.x >> 6;
  const int h = lane >> 5, lr = lane & 31;
  const int tile = blockIdx.x;
  const uint4* __restrict__ wb;
  const uint16_t* __restrict__ sb;
  float* yout;
  int R, ldy, NU, ldq, ldd, cntM, p0;
  const int* xrow = nullptr;
  if(GRP){
    /* the active count and this block's expert loaded together (act holds E entries: an index past the count reads
       an unused entry, not used) */
    const int nact = *ga.nact, e = ga.act[blockIdx.y];
    if((int)blockIdx.y >= nact) return;
    const uint8_t* base = ga.wexp[e];
    NU = ga.NU; R = ga.R;
    wb = (const uint4*)base;
    sb = (const uint16_t*)(base + (long long)kt_r8(R) * NU * 256);
    ldy = ga.ldy; ldq = ga.ldq; ldd = ga.ldd; cntM = ga.cnt[e]; p0 = ga.off[e]; xrow = ga.xrow;
    yout = ga.y;
  } else {
    NU = a.NU; R = a.mat[0].R;
    wb = (const uint4*)a.mat[0].codes;
    sb = a.mat[0].scales;
    ldy = a.mat[0].ldy; ldq = a.ldq; ldd = a.ldxs; cntM = a.M; p0 = 0;
    yout = a.mat[0].y;
  }
  const int S = kt_steps(NU);
  const int rg = tile * 4 + (lr >> 3), r = lr & 7, row = rg * KT_RG + r;
  const bool rok = row < R;
  int ks = wv, s_lo = 0, ns = 0;                                 /* the current slice and its steps (1 or 2) */
  auto set_slice = [&](int k){ ks = k; s_lo = k * S / KS; ns = (k + 1) * S / KS - s_lo; };
  set_slice(wv);
  const int nrows = GRP ? ga.nrows : cntM;

  /* a pass's loads, all unconditional (clamped) and issued together: the D scales of the slice's 16 units x 16
     tokens (to this wave's LDS region before the products, so the epilogue reads them there), and this lane's
     activations of the 16 units through a buffer resource over the input rows (lanes past the pass's tokens read at
     2^31, past the range, which gives zeros without a memory access; the launcher keeps the rows below 2^31 bytes) */
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)xq, (short)0, nrows * ldq, 0x00020000);
  float* xsl = (float*)(kt_lds + (size_t)KS * NT * 32 * 4) + (size_t)wv * 256;
  float xsv[4];
  uint4 xa[2 * KT_KL];
  /* the pass's input rows (the list indirection) first, the loads that need them after */
  int nrq[4], na = 0;
  auto ld_rows = [&](int t0){
    const int nt = min(NT, cntM - t0);
#pragma unroll
    for(int q = 0; q < 4; ++q){
      const int tl = (lane + 64 * q) & 15;
      const int pt = p0 + t0 + (tl < nt ? tl : 0);
      nrq[q] = xrow ? xrow[pt] : pt;
    }
    const int pe = p0 + t0 + (lr < nt ? lr : 0);
    na = xrow ? xrow[pe] : pe;
  };
  auto ld_pass = [&](int t0){
    const int nt = min(NT, cntM - t0);
#pragma unroll
    for(int q = 0; q < 4; ++q){
      const int idx = lane + 64 * q, n = idx >> 4;
      const int u = (s_lo + (n >> 3)) * KT_KL + (n & 7);
      xsv[q] = xd[(long long)nrq[q] * ldd + (u < NU ? u : 0)];
    }
    const uint32_t xo = lr < nt ? (uint32_t)(na * ldq + 16 * h) : (1u << 31);
#pragma unroll
    for(int n = 0; n < 2 * KT_KL; ++n){
      const int c = n >> 1, j = n & 1, u = (s_lo + j) * KT_KL + c;
      const int uu = (j < ns && u < NU) ? u : 0;
      xa[n] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, xo + uu * 32, 0, 0));
    }
  };
  /* the slice's 16 units in k-lane-major order (unconditional: a unit past the slice or the matrix reads offset 0) */
  uint4 wq[2][KT_KL];
  uint16_t hq[2][KT_KL];
  auto ld_w = [&](){
#pragma unroll
    for(int c = 0; c < KT_KL; ++c)
#pragma unroll
      for(int j = 0; j < 2; ++j){
        const int s = s_lo + j, u = s * KT_KL + c;
        const bool ok = rok && j < ns && u < NU;
        wq[j][c] = kt_ldnt(wb + (ok ? kt_widx(NU, rg, s, h, c, r) : 0));
        hq[j][c] = sb[ok ? kt_sidx(NU, rg, u, r) : 0];
      }
  };
  /* the slice's products for the pass at t0 into red[ks] */
  auto compute = [&](int t0){
#pragma unroll
    for(int q = 0; q < 4; ++q) xsl[lane + 64 * q] = xsv[q];
    kt_wave_sync();
    float part[NE], t01[NE], t23[NE], t45[NE], pend[NE];
#pragma unroll
    for(int e = 0; e < NE; ++e){ part[e] = 0.0f; t01[e] = 0.0f; t23[e] = 0.0f; t45[e] = 0.0f; pend[e] = 0.0f; }
#pragma unroll
    for(int c = 0; c < KT_KL; ++c){
      float chain[NE];
#pragma unroll
      for(int e = 0; e < NE; ++e) chain[e] = 0.0f;
#pragma unroll
      for(int j = 0; j < 2; ++j){
        const int s = s_lo + j, u = s * KT_KL + c;
        const bool uok = j < ns && u < NU;                      /* wave-uniform */
        const uint4 x = xa[2 * c + j];
        if(uok){
          const float d = rok ? kt_h2f(hq[j][c]) : 0.0f;
          const kt_v4i A = {(int)x.x, (int)x.y, (int)x.z, (int)x.w};
          const kt_v4i B = {(int)wq[j][c].x, (int)wq[j][c].y, (int)wq[j][c].z, (int)wq[j][c].w};
          const kt_v16i acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, (kt_v16i){}, 0, 0, 0);
#pragma unroll
          for(int e = 0; e < NE; ++e){
            const float sx = xsl[(j * 8 + c) * 16 + km_tok(e, lane)];
            chain[e] = fmaf((float)acc[e], d * sx, chain[e]);
            if(DBG){
              const int t = t0 + km_tok(e, lane);
              if(t < cntM && rok) dbg[((long long)(p0 + t) * R + row) * NU + u] = acc[e];
            }
          }
        }
      }
#pragma unroll
      for(int e = 0; e < NE; ++e){
        if(c == 0 || c == 2 || c == 4 || c == 6) pend[e] = chain[e];
        else if(c == 1) t01[e] = pend[e] + chain[e];
        else if(c == 3) t23[e] = t01[e] + (pend[e] + chain[e]);
        else if(c == 5) t45[e] = pend[e] + chain[e];
        else part[e] = t23[e] + (t45[e] + (pend[e] + chain[e]));
      }
    }
#pragma unroll
    for(int e = 0; e < NE; ++e) red[((size_t)ks * NT + km_tok(e, lane)) * 32 + lr] = part[e];
  };
  /* the pass's slice sums in slice order, by wave 0 */
  auto finish = [&](int t0){
    __syncthreads();
    if(wv == 0){
      float v[NE];
#pragma unroll
      for(int e = 0; e < NE; ++e) v[e] = red[(size_t)km_tok(e, lane) * 32 + lr];
      for(int k = 1; k < KS; ++k){
        float w[NE];
#pragma unroll
        for(int e = 0; e < NE; ++e) w[e] = red[((size_t)k * NT + km_tok(e, lane)) * 32 + lr];
#pragma unroll
        for(int e = 0; e < NE; ++e) v[e] += w[e];
      }
#pragma unroll
      for(int e = 0; e < NE; ++e){
        const int t = t0 + km_tok(e, lane);
        if(t < cntM && rok) yout[(long long)(p0 + t) * ldy + row] = v[e];
      }
    }
    __syncthreads();                                             /* red is rewritten by the next pass */
  };

  if(!MS){
    /* one slice a wave, its weights loaded once for every pass: the input rows of pass 0, then the weights
       (independent of them), then the pass's D and activations, so the weight stream overlaps the list
       indirection; each pass issues the next pass's loads before its slice sums */
    ld_rows(0);
    __builtin_amdgcn_sched_barrier(0);
    ld_w();
    __builtin_amdgcn_sched_barrier(0);
    ld_pass(0);
    for(int t0 = 0; t0 < cntM; t0 += NT){                        /* uniform: the block's list in passes */
      compute(t0);
      if(t0 + NT < cntM){ ld_rows(t0 + NT); ld_pass(t0 + NT); }  /* uniform: the next pass's loads in flight */
      finish(t0);
    }
  } else {
    /* several slices a wave, one after the other (each with its own weights, read again every pass: from L2
       after the first), so blocks are small and more of them share a CU's wave slots */
    for(int t0 = 0; t0 < cntM; t0 += NT){
      ld_rows(t0);
      for(int k = wv; k < KS; k += W){                           /* uniform */
        set_slice(k);
        ld_w();
        ld_pass(t0);
        compute(t0);
      }
      finish(t0);
    }
  }
}

#define KQ8(GRP, DBG, MS) template __global__ void k_q8_mma<GRP, DBG, MS>(const KtGemvArgs, const KtGroupedArgs, \
    const int8_t*, const float*, int32_t*, int);
KQ8(false, false, false) KQ8(false, true, false) KQ8(true, false, false) KQ8(true, true, false)
KQ8(true, false, true) KQ8(true, true, true)
#undef KQ8

#ifdef KT_TRACE
extern "C" int kt_trace_mma_read(void* host){
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(kt_trace_buf), sizeof(kt_trace_buf), 0, hipMemcpyDeviceToHost);
}
extern "C" int kt_trace_mma_enable(int on){
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(kt_trace_on), &on, sizeof(int), 0, hipMemcpyHostToDevice);
}
#endif
