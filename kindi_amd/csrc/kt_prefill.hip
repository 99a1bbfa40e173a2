/* kt_prefill.hip - the prefill product on the matrix cores (k_tc_mm2 tc_hip.cu:243-269, k_mm_g5q chunk.cu:858-918).

   Y[t][r] = sum_g fmaf((float)v(t, r, g), XS[t][g] * d[r][g], .) over the 128-column groups g in order, where
   v(t, r, g) = sum of t(r, c) q(t, c) over the group is an exact int32 from V_MFMA_I32_32X32X32_I8.

   Block: 256 threads (4 waves) own 128 tokens x 128 weight rows; wave (wt, wr) owns tokens 64 wt .., rows 64 wr ..
   as 2 x 2 MFMA tiles of 32 x 32. Per group: the block loads the 128 rows' packed trits (4 KB: one 16-byte load
   per thread, 32 lines of 128 bytes of the kt2 layout), unpacks them to signed int8 once (shift, mask, v_perm byte
   lookup) into LDS, stages the 128 tokens' int8 activations in LDS, and each wave runs 4 k-steps of 2 x 2 MFMAs.
   Two LDS stages and two register sets: the global loads of group g + 2 (through buffer resources: 32-bit offsets,
   out-of-range reads are zeros without a branch) are issued before group g's products, and group g + 1 is unpacked
   into the other stage after its epilogue, so one barrier a group separates the stages and every load has two
   groups of products to arrive. The MFMA A operand is the activations (rows = tokens), B the weights (columns =
   weight rows), so a lane's 16 accumulators share one weight row: its group scale is one register. After the group
   the int32 accumulators are scaled into fp32 accumulators (the reference expression, or with per-row scales
   fmaf(v, d, .) and XS[t] at the end) and cleared. Blocks take their tiles in the XCD order of kt_xcd_tile.

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

template <bool DBG, bool RS>   /* RS: per-row activation scales, Y[t][r] = XS[t][0] sum_g fmaf(v, d[r][g], .) */
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) k_tern_gemm(const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, int R, int NG, const int8_t* __restrict__ XQ, int ldq,
    const float* __restrict__ XS, int M, float* __restrict__ Y, uint16_t* __restrict__ Y16, int ldy,
    int32_t* __restrict__ dbg){
  /* two LDS stages: group g's operands are read while group g + 1's are written; one barrier a group */
  __shared__ __attribute__((aligned(16))) uint8_t Xl[2][PF_BT * PF_LD];
  __shared__ __attribute__((aligned(16))) uint8_t Wl[2][PF_BR * PF_LD];
  __shared__ float xs_l[2][2 * PF_BT];                          /* [PF_BT, 2 PF_BT): written, never read */

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, wt = wv >> 1, wr = wv & 1;
  int bx, by;
  kt_xcd_tile(blockIdx.x + blockIdx.y * gridDim.x, gridDim.x, gridDim.y, bx, by);
  const int r0 = bx * PF_BR, n0 = by * PF_BT;

  const int R8 = kt_r8(R);
  /* every global read goes through a buffer resource (a scalar base and a 32-bit offset a lane): an offset past the
     range reads zeros without a memory access or a branch. Zeros only reach accumulators of rows past R or tokens past
     M, which are never stored (the launcher keeps each buffer below 2^31 bytes, so 2^31 is past every range) */
  const uint32_t OOB = 1u << 31;
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)codes, (short)0, R8 * NG * 256, 0x00020000);
  const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc((void*)scales, (short)0, R8 * NG * 16, 0x00020000);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)XQ, (short)0, M * ldq, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)XS, (short)0, M * NG * 4, 0x00020000);
  /* this thread's weight chunk: row group r0/8 + (tid >> 4), half (tid >> 3) & 1, row tid & 7 (16 bytes = 64
     columns of one row); a unit's 128 rows are 32 chunks of 128 contiguous bytes */
  const int lrg = tid >> 4, lh = (tid >> 3) & 1, lr = tid & 7;
  const int grg = (r0 >> 3) + lrg;
  const int woff = (lrg * 8 + lr) * PF_LD + lh * 64;
  /* byte offset of the chunk of group g: wbase + lh nc(g) 128 + 2048 (g / 8) + 128 (g % 8), nc(g) the units of g's
     step (kt_widx) */
  const uint32_t wbase = grg < R8 ? (uint32_t)(grg * NG * 16 + lr) * 16 : OOB;

  /* this thread's activation chunk: token tid/2, 64 bytes at (tid&1)*64 (past M: out of range) */
  const int xt = tid >> 1, xh = tid & 1;
  const uint32_t xbase = (uint32_t)(n0 + xt) * (uint32_t)ldq + xh * 64;
  const int xoff = xt * PF_LD + xh * 64;
  const uint32_t sbase = tid < PF_BT ? (uint32_t)(n0 + tid) * NG * 4 : OOB;

  /* scales of this lane's two weight rows (columns of the 2 B tiles) */
  const int cr0 = r0 + wr * 64 + (lane & 31), cr1 = cr0 + 32;
  /* byte offsets of their scales of group 0 (group g: + 16 g) */
  const uint32_t hbase0 = (cr0 >> 3) < R8 ? (uint32_t)(((cr0 >> 3) * NG * 8 + (cr0 & 7)) * 2) : OOB;
  const uint32_t hbase1 = (cr1 >> 3) < R8 ? (uint32_t)(((cr1 >> 3) * NG * 8 + (cr1 & 7)) * 2) : OOB;

  /* the global loads of group g into registers (clamped: past the last group it is read again, so every group issues
     the same loads and the waits stay exact), and the unpack of a set into LDS stage b. Macros with named registers,
     not a struct by reference: the register sets must stay in registers */
#define KT_PF_LOADW(g, WC, H0, H1) do { \
    const int gg_ = (g) < NG ? (g) : NG - 1; \
    const int nc_ = NG - (gg_ & ~7) < 8 ? NG - (gg_ & ~7) : 8; \
    WC = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, wbase + (lh ? nc_ * 128 : 0), \
         (gg_ >> 3) * 2048 + (gg_ & 7) * 128, 2)); \
    H0 = __builtin_amdgcn_raw_buffer_load_b16(rh, hbase0, gg_ * 16, 0); \
    H1 = __builtin_amdgcn_raw_buffer_load_b16(rh, hbase1, gg_ * 16, 0); \
  } while(0)
#define KT_PF_LOADX(g, X0, X1, X2, X3, XSV) do { \
    const int gg_ = (g) < NG ? (g) : NG - 1; \
    X0 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, xbase, gg_ * 128, 0)); \
    X1 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, xbase + 16, gg_ * 128, 0)); \
    X2 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, xbase + 32, gg_ * 128, 0)); \
    X3 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, xbase + 48, gg_ * 128, 0)); \
    if(!RS) XSV = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, sbase, gg_ * 4, 0)); } while(0)
  auto store = [&](const uint4 wc, const uint4 x0, const uint4 x1, const uint4 x2, const uint4 x3, float xsv, int b){
    /* unpack: word j of the chunk = columns 16j .. +15 of the half; slot s = columns 16j + 4s .. +3 */
    const uint32_t ww[4] = {wc.x, wc.y, wc.z, wc.w};
#pragma unroll
    for(int j = 0; j < 4; ++j){
      uint4 o;
      o.x = kt_trits(ww[j] & 0x03030303u);
      o.y = kt_trits((ww[j] >> 2) & 0x03030303u);
      o.z = kt_trits((ww[j] >> 4) & 0x03030303u);
      o.w = kt_trits((ww[j] >> 6) & 0x03030303u);
      *(uint4*)(Wl[b] + woff + 16 * j) = o;
    }
    *(uint4*)(Xl[b] + xoff) = x0;
    *(uint4*)(Xl[b] + xoff + 16) = x1;
    *(uint4*)(Xl[b] + xoff + 32) = x2;
    *(uint4*)(Xl[b] + xoff + 48) = x3;
    if(!RS) xs_l[b][tid] = xsv;
  };

  float acc[2][2][16];
#pragma unroll
  for(int i = 0; i < 2; ++i)
#pragma unroll
    for(int j = 0; j < 2; ++j)
#pragma unroll
      for(int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  /* group g's products and epilogue from LDS stage g % 2 with row scales d0, d1 */
  auto prod = [&](int g, float d0, float d1){
    const int b = g & 1;
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
    /* group epilogue: acc += (float)v * (XS[t][g] * d[r][g]), or acc += (float)v * d[r][g] (RS) */
#pragma unroll
    for(int i = 0; i < 2; ++i)
#pragma unroll
      for(int e = 0; e < 16; ++e){
        const int tl = wt * 64 + i * 32 + (e & 3) + 8 * (e >> 2) + 4 * (lane >> 5);
        if(RS){
          acc[i][0][e] = fmaf((float)c[i][0][e], d0, acc[i][0][e]);
          acc[i][1][e] = fmaf((float)c[i][1][e], d1, acc[i][1][e]);
        } else {
          const float xs = xs_l[b][tl];
          acc[i][0][e] = fmaf((float)c[i][0][e], xs * d0, acc[i][0][e]);
          acc[i][1][e] = fmaf((float)c[i][1][e], xs * d1, acc[i][1][e]);
        }
        if(DBG){
          const int t = n0 + tl;
          if(t < M){
            if(cr0 < R) dbg[((long long)t * R + cr0) * NG + g] = c[i][0][e];
            if(cr1 < R) dbg[((long long)t * R + cr1) * NG + g] = c[i][1][e];
          }
        }
      }
  };

  /* every global load two groups ahead, in two register sets: at the start of group g the set holding g + 1 is
     landing and g + 2 is issued into the other; after group g's products, g + 1 is unpacked into the other LDS
     stage */
  uint4 wa, wb, xa0, xa1, xa2, xa3, xb0, xb1, xb2, xb3;
  uint16_t ha0, ha1, hb0, hb1;
  float xsa = 0.0f, xsb = 0.0f, d0, d1;
  KT_PF_LOADW(0, wa, ha0, ha1);
  KT_PF_LOADX(0, xa0, xa1, xa2, xa3, xsa);
  KT_PF_LOADW(1, wb, hb0, hb1);
  KT_PF_LOADX(1, xb0, xb1, xb2, xb3, xsb);
  store(wa, xa0, xa1, xa2, xa3, xsa, 0);
  d0 = kt_h2f(ha0); d1 = kt_h2f(ha1);
  __syncthreads();
  /* step: group g; set S holds g + 1, set T takes g + 2 */
#define KT_PF_STEP(g, WS, HS0, HS1, XS0, XS1, XS2, XS3, XSS, WT_, HT0, HT1, XT0, XT1, XT2, XT3, XST) do { \
    KT_PF_LOADW((g) + 2, WT_, HT0, HT1); \
    KT_PF_LOADX((g) + 2, XT0, XT1, XT2, XT3, XST); \
    prod((g), d0, d1); \
    store(WS, XS0, XS1, XS2, XS3, XSS, ((g) & 1) ^ 1); \
    d0 = kt_h2f(HS0); d1 = kt_h2f(HS1); \
    __syncthreads(); } while(0)
  int g = 0;
  for(; g + 2 <= NG; g += 2){
    KT_PF_STEP(g, wb, hb0, hb1, xb0, xb1, xb2, xb3, xsb, wa, ha0, ha1, xa0, xa1, xa2, xa3, xsa);
    KT_PF_STEP(g + 1, wa, ha0, ha1, xa0, xa1, xa2, xa3, xsa, wb, hb0, hb1, xb0, xb1, xb2, xb3, xsb);
  }
  if(g < NG) prod(g, d0, d1);
#undef KT_PF_STEP
#undef KT_PF_LOADW
#undef KT_PF_LOADX
  /* store. fp16 rows 16-byte aligned (ldy % 8 == 0): each wave stages its 64 tokens x 64 rows in LDS (the X stages
     are free once every wave is past its last group), token rows at a 16-byte-padded pitch, and writes 16 bytes a
     lane, whole token rows in contiguous runs (8 store instructions in place of 64 two-byte ones). Else, and fp32,
     lanes of one register write 32 consecutive rows of one token. */
  const bool v16 = Y16 && (uintptr_t)Y16 % 16 == 0 && ldy % 8 == 0;
  if(v16) __syncthreads();
#pragma unroll
  for(int i = 0; i < 2; ++i)
#pragma unroll
    for(int e = 0; e < 16; ++e){
      const int t = n0 + wt * 64 + i * 32 + (e & 3) + 8 * (e >> 2) + 4 * (lane >> 5);
      if(t < M){
        const float xr = RS ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (uint32_t)t * NG * 4, 0, 0))
                            : 1.0f;
        float y0 = RS ? acc[i][0][e] * xr : acc[i][0][e], y1 = RS ? acc[i][1][e] * xr : acc[i][1][e];
        /* the fp32 values, then fp16 (two roundings): not folded into a mixed-precision instruction */
        asm volatile("" : "+v"(y0), "+v"(y1));
        if(cr0 < R){
          if(Y) Y[(long long)t * ldy + cr0] = y0;
          if(Y16 && !v16) Y16[(long long)t * ldy + cr0] = __half_as_ushort(__float2half_rn(y0));
        }
        if(cr1 < R){
          if(Y) Y[(long long)t * ldy + cr1] = y1;
          if(Y16 && !v16) Y16[(long long)t * ldy + cr1] = __half_as_ushort(__float2half_rn(y1));
        }
        if(v16){
          const int lt = i * 32 + (e & 3) + 8 * (e >> 2) + 4 * (lane >> 5);
          uint16_t* o = (uint16_t*)(&Xl[0][0] + wv * 64 * PF_LD + lt * PF_LD) + (lane & 31);
          o[0] = __half_as_ushort(__float2half_rn(y0));
          o[32] = __half_as_ushort(__float2half_rn(y1));
        }
      }
    }
  if(v16){
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int tw0 = n0 + wt * 64, rw0 = r0 + wr * 64;
#pragma unroll
    for(int k = 0; k < 8; ++k){
      const int lt = (lane >> 3) + 8 * k, t = tw0 + lt, row = rw0 + 8 * (lane & 7);
      if(t < M && row < R){
        const uint4 v = *(const uint4*)(&Xl[0][0] + wv * 64 * PF_LD + lt * PF_LD + 16 * (lane & 7));
        uint16_t* dst = Y16 + (long long)t * ldy + row;
        if(row + 8 <= R) *(uint4*)dst = v;
        else {                                                     /* the last rows of a ragged R */
          const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for(int q = 0; q < 8; ++q)
            if(row + q < R) dst[q] = (uint16_t)(vw[q >> 1] >> (16 * (q & 1)));
        }
      }
    }
  }
}

#define KT_TG(DBG, RS) template __global__ void k_tern_gemm<DBG, RS>(const uint32_t*, const uint16_t*, int, int, \
    const int8_t*, int, const float*, int, float*, uint16_t*, int, int32_t*);
KT_TG(false, false) KT_TG(true, false) KT_TG(false, true) KT_TG(true, true)

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
  int bx, by;
  kt_xcd_tile(blockIdx.x + blockIdx.y * gridDim.x, gridDim.x, gridDim.y, bx, by);
  const int r0 = bx * BR, n0 = by * BT;
  const int R8 = kt_r8(R);

  /* every global read through a buffer resource: an offset past the range (2^31; the launcher keeps the buffers
     below it) reads zeros without a memory access or a branch, and zeros only reach rows past R or tokens past M,
     which are never stored */
  const uint32_t OOB = 1u << 31;
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)codes, (short)0, R8 * NG * 256, 0x00020000);
  const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc((void*)scales, (short)0, R8 * NG * 16, 0x00020000);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)XQ, (short)0, M * ldq, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)XS, (short)0, M * NG * 4, 0x00020000);
  /* activations: token tid / 4 of the block, 32 bytes at (tid % 4) 32 of each group */
  const int xt = tid >> 2, xq = tid & 3;
  const uint32_t xbase = (uint32_t)(n0 + xt) * (uint32_t)ldq + xq * 32;
  const int xdst = xt * PF_LD + xq * 32;
  /* packed trits: word tid of the group's NW (chunk tid / 4 = (row group, half, row), word tid % 4) */
  const bool wown = tid < NW;
  const int ch = (tid >> 2) & (2 * BR - 1), wj = tid & 3;
  const int lrg = ch >> 4, lh = (ch >> 3) & 1, lr = ch & 7;
  const int grg = (r0 >> 3) + lrg;
  const uint32_t wbase = grg < R8 ? (uint32_t)(grg * NG * 16 + lr) * 16 + wj * 4 : OOB;
  const int wdst = (lrg * 8 + lr) * PF_LD + lh * 64 + 16 * wj;
  /* this lane's tile: tokens 32 wt + .., weight row cr (its scale row clamped to a real one) */
  const int cr = r0 + 32 * wr + (lane & 31);
  const uint32_t hbase = cr < R8 * KT_RG ? (uint32_t)(((cr >> 3) * NG * 8 + (cr & 7)) * 2) : OOB;

  /* the global loads of group g (clamped: past the last group it is read again) into registers X0 X1 W H; the
     LDS stores of such a set into stage b. Macros with named registers, not a struct: the three sets must stay in
     registers (a struct by reference let the compiler merge the three steps behind a pointer select) */
#define KT_RS1_LOAD(g, X0, X1, W, H) do { \
    const int gg_ = (g) < NG ? (g) : NG - 1; \
    const int nc_ = NG - (gg_ & ~7) < 8 ? NG - (gg_ & ~7) : 8; \
    X0 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, xbase, gg_ * 128, 0)); \
    X1 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, xbase + 16, gg_ * 128, 0)); \
    W = __builtin_amdgcn_raw_buffer_load_b32(rw, wbase + (lh ? nc_ * 128 : 0), (gg_ >> 3) * 2048 + (gg_ & 7) * 128, 2); \
    H = __builtin_amdgcn_raw_buffer_load_b16(rh, hbase, gg_ * 16, 0); } while(0)
  auto store = [&](const uint4 x0, const uint4 x1, const uint32_t wraw, int b){
    *(uint4*)(Xl[b] + xdst) = x0;
    *(uint4*)(Xl[b] + xdst + 16) = x1;
    if(wown){
      const uint32_t w = wraw;                                  /* rows past the matrix: zeros, never stored */
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
      float y = acc[e] * __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (uint32_t)t * NG * 4, 0, 0));
      asm volatile("" : "+v"(y));                                /* fp32, then fp16: two roundings */
      if(Y) Y[(long long)t * ldy + cr] = y;
      if(Y16) Y16[(long long)t * ldy + cr] = __half_as_ushort(__float2half_rn(y));
    }
  }
}

#define KT_RS1(WT, WR, PD, DBG) template __global__ void k_tern_gemm_rs1<WT, WR, PD, DBG>(const uint32_t*, \
    const uint16_t*, int, int, const int8_t*, int, const float*, int, float*, uint16_t*, int, int32_t*);
KT_RS1(4, 2, 3, false) KT_RS1(4, 2, 3, true)

