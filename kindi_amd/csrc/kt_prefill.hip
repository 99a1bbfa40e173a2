/* kt_prefill.hip - the prefill product on the matrix cores (k_tc_mm2 tc_hip.cu:243-269, k_mm_g5q chunk.cu:858-918).

   Y[t][r] = sum_g fmaf((float)v(t, r, g), XS[t][g] * d[r][g], .) over the 128-column groups g in order, where
   v(t, r, g) = sum of t(r, c) q(t, c) over the group is an exact int32 from V_MFMA_I32_32X32X32_I8.

   Block: 256 threads (4 waves) own 128 tokens x 128 weight rows; wave (wt, wr) owns tokens 64 wt .., rows 64 wr ..
   as 2 x 2 MFMA tiles of 32 x 32. Per group: the block loads the 128 rows' packed trits (4 KB: one 16-byte load
   per thread, 32 lines of 128 bytes of the kt2 layout), unpacks them to signed int8 once (shift, mask, v_perm byte
   lookup) into LDS, stages the 128 tokens' int8 activations in LDS, and each wave runs 4 k-steps of 2 x 2 MFMAs.
   Two LDS stages: the loads of group g + 1 are issued before group g's products and unpacked into the other stage
   after its epilogue, so one barrier a group separates the stages and the memory latency overlaps the products. The
   MFMA A operand is the activations (rows = tokens), B the weights (columns = weight rows), so a lane's 16
   accumulators share one weight row: its group scale is one register. After the group the int32 accumulators are
   scaled into fp32 accumulators in the reference expression and cleared.

   MFMA 32x32x32 i8 register layouts on gfx950 (measured): A lane l holds row l % 32, k = 16 (l / 32) .. +15;
   B lane l holds column l % 32, the same k; D lane l register i holds column l % 32, row (i % 4) + 8 (i / 4) +
   4 (l / 32). */
#include "kt_common.h"

typedef int kt_v4i __attribute__((ext_vector_type(4)));
typedef int kt_v16i __attribute__((ext_vector_type(16)));

#define PF_BT 128                     /* tokens per block */
#define PF_BR 128                     /* weight rows per block */
#define PF_LD 144                     /* LDS row stride in bytes (128 + 16: rows land on different banks) */

/* 4 digits (0/1/2, one per byte) -> 4 signed trits (-1/0/+1): byte lookup in 0x000100FF */
__device__ __forceinline__ uint32_t kt_trits(uint32_t dig){ return __builtin_amdgcn_perm(0x000100FFu, 0x000100FFu, dig); }

template <bool DBG>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) k_tern_gemm(const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, int R, int NG, const int8_t* __restrict__ XQ, int ldq,
    const float* __restrict__ XS, int M, float* __restrict__ Y, uint16_t* __restrict__ Y16, int ldy,
    int32_t* __restrict__ dbg){
  /* two LDS stages: group g's operands are read while group g + 1's are written; one barrier a group */
  __shared__ __attribute__((aligned(16))) uint8_t Xl[2][PF_BT * PF_LD];
  __shared__ __attribute__((aligned(16))) uint8_t Wl[2][PF_BR * PF_LD];
  __shared__ float xs_l[2][PF_BT];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, wt = wv >> 1, wr = wv & 1;
  const int r0 = blockIdx.x * PF_BR, n0 = blockIdx.y * PF_BT;

  const int R8 = kt_r8(R);
  /* this thread's weight chunk: row group r0/8 + (tid >> 4), half (tid >> 3) & 1, row tid & 7 (16 bytes = 64
     columns of one row); a unit's 128 rows are 32 chunks of 128 contiguous bytes */
  const int lrg = tid >> 4, lh = (tid >> 3) & 1, lr = tid & 7;
  const int grg = (r0 >> 3) + lrg;
  const bool wvalid = grg < R8;
  const uint4* __restrict__ wsrc = (const uint4*)codes;
  const int woff = (lrg * 8 + lr) * PF_LD + lh * 64;

  /* this thread's activation chunk: token tid/2, 64 bytes at (tid&1)*64 */
  const int xt = tid >> 1, xh = tid & 1;
  const bool xvalid = n0 + xt < M;
  const int8_t* __restrict__ xsrc = XQ + (long long)(n0 + (xvalid ? xt : 0)) * ldq + xh * 64;
  const int xoff = xt * PF_LD + xh * 64;

  /* scales of this lane's two weight rows (columns of the 2 B tiles) */
  const int cr0 = r0 + wr * 64 + (lane & 31), cr1 = cr0 + 32;
  const int crg0 = cr0 >> 3, crg1 = cr1 >> 3;
  const bool c0v = (cr0 >> 3) < R8, c1v = (cr1 >> 3) < R8;

  /* the global loads of one group (registers), then their unpack into LDS stage b */
  struct Grp { uint4 wc; uint4 xv[4]; uint16_t h0, h1; float xs; };
  auto load = [&](int g, Grp& q){
    q.wc = wvalid ? kt_ldnt(wsrc + kt_widx(NG, grg, g >> 3, lh, g & 7, lr))
                  : make_uint4(0x55555555u, 0x55555555u, 0x55555555u, 0x55555555u);
#pragma unroll
    for(int k = 0; k < 4; ++k) q.xv[k] = xvalid ? ((const uint4*)(xsrc + g * 128))[k] : make_uint4(0u, 0u, 0u, 0u);
    q.h0 = c0v ? scales[kt_sidx(NG, crg0, g, cr0 & 7)] : (uint16_t)0;
    q.h1 = c1v ? scales[kt_sidx(NG, crg1, g, cr1 & 7)] : (uint16_t)0;
    q.xs = (tid < PF_BT && n0 + tid < M) ? XS[(long long)(n0 + tid) * NG + g] : 0.0f;
  };
  auto store = [&](const Grp& q, int b){
    /* unpack: word j of the chunk = columns 16j .. +15 of the half; slot s = columns 16j + 4s .. +3 */
    const uint32_t ww[4] = {q.wc.x, q.wc.y, q.wc.z, q.wc.w};
#pragma unroll
    for(int j = 0; j < 4; ++j){
      uint4 o;
      o.x = kt_trits(ww[j] & 0x03030303u);
      o.y = kt_trits((ww[j] >> 2) & 0x03030303u);
      o.z = kt_trits((ww[j] >> 4) & 0x03030303u);
      o.w = kt_trits((ww[j] >> 6) & 0x03030303u);
      *(uint4*)(Wl[b] + woff + 16 * j) = o;
    }
#pragma unroll
    for(int k = 0; k < 4; ++k) *(uint4*)(Xl[b] + xoff + 16 * k) = q.xv[k];
    if(tid < PF_BT) xs_l[b][tid] = q.xs;
  };

  float acc[2][2][16];
#pragma unroll
  for(int i = 0; i < 2; ++i)
#pragma unroll
    for(int j = 0; j < 2; ++j)
#pragma unroll
      for(int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  Grp cur, nxt;
  load(0, cur);
  store(cur, 0);
  float d0 = kt_h2f(cur.h0), d1 = kt_h2f(cur.h1);
  __syncthreads();
  for(int g = 0; g < NG; ++g){
    const int b = g & 1;
    if(g + 1 < NG) load(g + 1, nxt);                          /* in flight during this group's products */
    kt_v16i c[2][2];
#pragma unroll
    for(int i = 0; i < 2; ++i)
#pragma unroll
      for(int j = 0; j < 2; ++j)
#pragma unroll
        for(int e = 0; e < 16; ++e) c[i][j][e] = 0;
#pragma unroll
    for(int ks = 0; ks < 4; ++ks){
      const int koff = ks * 32 + (lane >> 5) * 16;
      kt_v4i A[2], B[2];
#pragma unroll
      for(int i = 0; i < 2; ++i) A[i] = *(const kt_v4i*)(Xl[b] + (wt * 64 + i * 32 + (lane & 31)) * PF_LD + koff);
#pragma unroll
      for(int j = 0; j < 2; ++j) B[j] = *(const kt_v4i*)(Wl[b] + (wr * 64 + j * 32 + (lane & 31)) * PF_LD + koff);
#pragma unroll
      for(int i = 0; i < 2; ++i)
#pragma unroll
        for(int j = 0; j < 2; ++j) c[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[i], B[j], c[i][j], 0, 0, 0);
    }
    /* group epilogue: acc += (float)v * (XS[t][g] * d[r][g]) */
#pragma unroll
    for(int i = 0; i < 2; ++i)
#pragma unroll
      for(int e = 0; e < 16; ++e){
        const int tl = wt * 64 + i * 32 + (e & 3) + 8 * (e >> 2) + 4 * (lane >> 5);
        const float xs = xs_l[b][tl];
        acc[i][0][e] = fmaf((float)c[i][0][e], xs * d0, acc[i][0][e]);
        acc[i][1][e] = fmaf((float)c[i][1][e], xs * d1, acc[i][1][e]);
        if(DBG){
          const int t = n0 + tl;
          if(t < M){
            if(cr0 < R) dbg[((long long)t * R + cr0) * NG + g] = c[i][0][e];
            if(cr1 < R) dbg[((long long)t * R + cr1) * NG + g] = c[i][1][e];
          }
        }
      }
    if(g + 1 < NG){
      store(nxt, b ^ 1);                                        /* stage b ^ 1 was last read in group g - 1 */
      d0 = kt_h2f(nxt.h0);
      d1 = kt_h2f(nxt.h1);
    }
    __syncthreads();
  }
  /* store: lanes of one register write 32 consecutive rows of one token */
#pragma unroll
  for(int i = 0; i < 2; ++i)
#pragma unroll
    for(int e = 0; e < 16; ++e){
      const int t = n0 + wt * 64 + i * 32 + (e & 3) + 8 * (e >> 2) + 4 * (lane >> 5);
      if(t < M){
        if(cr0 < R){
          if(Y) Y[(long long)t * ldy + cr0] = acc[i][0][e];
          if(Y16) Y16[(long long)t * ldy + cr0] = __half_as_ushort(__float2half_rn(acc[i][0][e]));
        }
        if(cr1 < R){
          if(Y) Y[(long long)t * ldy + cr1] = acc[i][1][e];
          if(Y16) Y16[(long long)t * ldy + cr1] = __half_as_ushort(__float2half_rn(acc[i][1][e]));
        }
      }
    }
}

template __global__ void k_tern_gemm<false>(const uint32_t*, const uint16_t*, int, int, const int8_t*, int, const float*,
                                            int, float*, uint16_t*, int, int32_t*);
template __global__ void k_tern_gemm<true>(const uint32_t*, const uint16_t*, int, int, const int8_t*, int, const float*,
                                           int, float*, uint16_t*, int, int32_t*);

/* ------------------------------------------------------------------ per-row activation scales
   The prefill product when the activations are quantized per token (kt_quant_q8 per_row: one XS a token, the
   quantization BASELINE's prefill config names): XS factors out of the group sum, so
     Y[t][r] = XS[t] * sum_g fmaf((float)v(t, r, g), d[r][g], .)      (groups in order)
   and the per-group epilogue is two VALU operations per element (convert, fma) instead of three. v(t, r, g) is the
   same exact int32 as above. One 32 x 32 tile a wave and WT x WR waves a block (32 WT tokens x 32 WR rows): small
   blocks, for matrices whose row count leaves the 128 x 128 kernel's grid short of the CUs. Both operands go through
   LDS (two stages, one barrier a group); every thread's global loads of group g + PD (32 bytes of activations, one
   word of packed trits, its tile column's scale) are issued PD groups before the group is stored to LDS, so the
   memory latency is covered by PD - 1 groups of products. The loads are unconditional (past the last group they
   read it again), so the loop issues the same loads every group. */
template <int WT, int WR, int PD, bool DBG>
__global__ void __launch_bounds__(64 * WT * WR) __attribute__((amdgpu_waves_per_eu(4))) k_tern_gemm_rs1(const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, int R, int NG, const int8_t* __restrict__ XQ, int ldq,
    const float* __restrict__ XS, int M, float* __restrict__ Y, uint16_t* __restrict__ Y16, int ldy,
    int32_t* __restrict__ dbg){
  constexpr int NT = 64 * WT * WR, BT = 32 * WT, BR = 32 * WR, NW = BR * 8;
  static_assert(NT == BT * 4 && NW <= NT, "one activation quarter-row and at most one packed word a thread");
  __shared__ __attribute__((aligned(16))) uint8_t Xl[2][BT * PF_LD];
  __shared__ __attribute__((aligned(16))) uint8_t Wl[2][BR * PF_LD];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, wt = wv / WR, wr = wv % WR;
  const int r0 = blockIdx.x * BR, n0 = blockIdx.y * BT;
  const int R8 = kt_r8(R);

  /* activations: token tid / 4 of the block, 32 bytes at (tid % 4) 32 of each group (clamped to a real row) */
  const int xt = tid >> 2, xq = tid & 3;
  const int8_t* xsrc = XQ + (long long)(n0 + xt < M ? n0 + xt : M - 1) * ldq + xq * 32;
  const int xdst = xt * PF_LD + xq * 32;
  /* packed trits: word tid of the group's NW (chunk tid / 4 = (row group, half, row), word tid % 4) */
  const bool wown = tid < NW;
  const int ch = (tid >> 2) & (2 * BR - 1), wj = tid & 3;
  const int lrg = ch >> 4, lh = (ch >> 3) & 1, lr = ch & 7;
  const int grg = (r0 >> 3) + lrg;
  const bool wvalid = grg < R8;
  const int wdst = (lrg * 8 + lr) * PF_LD + lh * 64 + 16 * wj;
  /* this lane's tile: tokens 32 wt + .., weight row cr (its scale row clamped to a real one) */
  const int cr = r0 + 32 * wr + (lane & 31);
  const int srow = cr < R8 * KT_RG ? cr : 0;

  /* the global loads of group g (clamped: past the last group it is read again) into registers X0 X1 W H; the
     LDS stores of such a set into stage b. Macros with named registers, not a struct: the three sets must stay in
     registers (a struct by reference let the compiler merge the three steps behind a pointer select) */
#define KT_RS1_LOAD(g, X0, X1, W, H) do { \
    const int gg_ = (g) < NG ? (g) : NG - 1; \
    const uint4* xp_ = (const uint4*)(xsrc + gg_ * 128); \
    X0 = xp_[0]; X1 = xp_[1]; \
    W = codes[wvalid ? kt_widx(NG, grg, gg_ >> 3, lh, gg_ & 7, lr) * 4 + wj : 0]; \
    H = scales[kt_sidx(NG, srow >> 3, gg_, srow & 7)]; } while(0)
  auto store = [&](const uint4 x0, const uint4 x1, const uint32_t wraw, int b){
    *(uint4*)(Xl[b] + xdst) = x0;
    *(uint4*)(Xl[b] + xdst + 16) = x1;
    if(wown){
      const uint32_t w = wvalid ? wraw : 0x55555555u;           /* rows past the matrix: digit 1, trit 0 */
      uint4 o;
      o.x = kt_trits(w & 0x03030303u);
      o.y = kt_trits((w >> 2) & 0x03030303u);
      o.z = kt_trits((w >> 4) & 0x03030303u);
      o.w = kt_trits((w >> 6) & 0x03030303u);
      *(uint4*)(Wl[b] + wdst) = o;
    }
  };

  float acc[16];
#pragma unroll
  for(int e = 0; e < 16; ++e) acc[e] = 0.0f;
  float dcur;
  {
    uint4 x0, x1;
    uint32_t w;
    uint16_t h;
    KT_RS1_LOAD(0, x0, x1, w, h);
    store(x0, x1, w, 0);
    dcur = kt_h2f(h);
  }
  /* group g: products and epilogue from stage g % 2 */
  auto prod = [&](int g){
    const int b = g & 1;
    kt_v16i c;
#pragma unroll
    for(int e = 0; e < 16; ++e) c[e] = 0;
#pragma unroll
    for(int ks = 0; ks < 4; ++ks){
      const int koff = ks * 32 + (lane >> 5) * 16;
      const kt_v4i A = *(const kt_v4i*)(Xl[b] + (32 * wt + (lane & 31)) * PF_LD + koff);
      const kt_v4i B = *(const kt_v4i*)(Wl[b] + (32 * wr + (lane & 31)) * PF_LD + koff);
      c = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, c, 0, 0, 0);
    }
#pragma unroll
    for(int e = 0; e < 16; ++e){
      acc[e] = fmaf((float)c[e], dcur, acc[e]);
      if(DBG){
        const int t = n0 + 32 * wt + (e & 3) + 8 * (e >> 2) + 4 * (lane >> 5);
        if(t < M && cr < R) dbg[((long long)t * R + cr) * NG + g] = c[e];
      }
    }
  };
  /* one group, then group g + 1 (loaded PD groups ago, in set S) into the other stage and g + 1 + PD into set S */
#define KT_RS1_STEP(g, X0, X1, W, H) do { \
    prod(g); \
    store(X0, X1, W, ((g) & 1) ^ 1); \
    dcur = kt_h2f(H); \
    KT_RS1_LOAD((g) + 1 + PD, X0, X1, W, H); \
    __syncthreads(); } while(0)
  static_assert(PD == 3, "three prefetch sets");
  uint4 xa0, xa1, xb0, xb1, xc0, xc1;
  uint32_t wa, wb, wc;
  uint16_t ha, hb, hc;
  KT_RS1_LOAD(1, xa0, xa1, wa, ha);
  KT_RS1_LOAD(2, xb0, xb1, wb, hb);
  KT_RS1_LOAD(3, xc0, xc1, wc, hc);
  __syncthreads();
  int g = 0;
  for(; g + 3 <= NG; g += 3){                                    /* the same loads every group: exact waits */
    KT_RS1_STEP(g, xa0, xa1, wa, ha);
    KT_RS1_STEP(g + 1, xb0, xb1, wb, hb);
    KT_RS1_STEP(g + 2, xc0, xc1, wc, hc);
  }
  if(g < NG) KT_RS1_STEP(g, xa0, xa1, wa, ha);
  if(g + 1 < NG) KT_RS1_STEP(g + 1, xb0, xb1, wb, hb);
#undef KT_RS1_STEP
#undef KT_RS1_LOAD
#pragma unroll
  for(int e = 0; e < 16; ++e){
    const int t = n0 + 32 * wt + (e & 3) + 8 * (e >> 2) + 4 * (lane >> 5);
    if(t < M && cr < R){
      const float y = acc[e] * XS[(long long)t * NG];
      if(Y) Y[(long long)t * ldy + cr] = y;
      if(Y16) Y16[(long long)t * ldy + cr] = __half_as_ushort(__float2half_rn(y));
    }
  }
}

#define KT_RS1(WT, WR, PD, DBG) template __global__ void k_tern_gemm_rs1<WT, WR, PD, DBG>(const uint32_t*, \
    const uint16_t*, int, int, const int8_t*, int, const float*, int, float*, uint16_t*, int, int32_t*);
KT_RS1(4, 2, 3, false) KT_RS1(4, 2, 3, true)

