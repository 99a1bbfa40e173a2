/* kt_prefill8.hip - the prefill product over an int8 copy of the trits (kt_tern_expand + kt_tern_gemm8).

   k_tern_expand writes the signed trits t = d - 1 of a kt2 matrix as int8 in natural order, W8 [8 R8][C] (rows padded
   to the kt2 row groups). The product then has nothing to unpack: both operands reach LDS by DMA
   (buffer_load_dwordx4 ... lds: no registers, no LDS store instructions), and the waves only read LDS, run the
   matrix cores and the per-group epilogue. The numbers are those of k_tern_gemm with per-row activation scales:
     Y[t][r] = XS[t] * sum_g fmaf((float)v(t, r, g), d[r][g], .)      (groups in order)
   with v(t, r, g) the exact int32 group value (k_mm_g5q's int8 trits, chunk.cu:836-918; the reference expression's
   per-group value, tc_hip.cu:171).

   k_tern_gemm8: 512 threads (8 waves) own 128 tokens x 256 weight rows; wave (wt, wr) = (w & 1, w >> 1) owns tokens
   64 wt .., rows 64 wr .. as 2 x 2 tiles of V_MFMA_I32_32X32X32_I8. Three LDS stages of one 128-column group (16 KB
   of activations, 32 KB of trits, 512 bytes of row scales): each wave issues the DMA of group g + 2 (7 instructions)
   right after the barrier that opens group g, so every group's operands have two groups of products to arrive. The
   DMAs are asm (the compiler would wait for all of them before any LDS read) and counted by hand: a wave's vector
   memory instructions in the loop are exactly its 7 DMAs a group, so vmcnt(7) at the top of group g leaves only
   group g + 1's in flight. LDS rows are 128 bytes with the 16-byte chunk c of row r at chunk position
   c ^ ((r >> 1) & 7): 16 lanes reading one chunk of 16 consecutive rows then touch all 64 banks once.
   Two sets of int32 accumulators: group g's MFMAs run while group g - 1's epilogue is applied, written out in issue
   order (each MFMA followed by 8 epilogue VALU operations; on gfx950 a wave issues in order, and the VALU work
   overlaps an MFMA only when it sits behind it in the stream). One block a CU (its 145 KB of LDS) takes tiles
   blockIdx.x, + gridDim.x, ...; a tile's outputs go out through LDS as 16-byte token rows before the next tile's
   first DMAs.
   Measured on MI355X (config 2, M = 2048, fp16 out, against k_tern_gemm on the packed trits): gate/up [12288 x 4096]
   131 against 199 us, down [4096 x 12288] 128 against 172 us (with two-byte stores straight from the accumulators:
   175 and 142 us). Below one block a CU (M = 512) the packed-trit kernels are faster and kt_tern_gemm8 runs them. */
#include "kt_common.h"

typedef int kt8_v4i __attribute__((ext_vector_type(4)));
typedef int kt8_v16i __attribute__((ext_vector_type(16)));
#define KT_L3 __attribute__((address_space(3)))

#define P8_BT 128                     /* tokens a block */
#define P8_BR 256                     /* weight rows a block */
#define P8_A (P8_BT * 128)            /* a stage's activations */
#define P8_W (P8_BR * 128)            /* a stage's trits */
#define P8_S (P8_BR * 2)              /* a stage's row scales (fp16) */
#define P8_STAGE (P8_A + P8_W + P8_S)
#define P8_NS 3                       /* stages */
#define P8_DMA 7                      /* DMA instructions a wave a group: 2 activation, 4 trit, 1 scale */

/* ------------------------------------------------------------------ the int8 copy */
/* one thread a kt2 chunk (16 bytes: 64 columns of one row) -> 64 int8 trits at their natural columns; consecutive
   threads read consecutive chunks (the 8 rows of a row group, then the next half unit) */
extern "C" __global__ void __launch_bounds__(256) k_tern_expand(const uint4* __restrict__ codes, int NU, long long nq,
                                                                 int C, int8_t* __restrict__ W8){
  const long long q = (long long)blockIdx.x * 256 + threadIdx.x;
  if(q >= nq) return;
  const long long rg = q / (NU * 16);
  const int rem = (int)(q - rg * NU * 16), s = rem >> 7, idx = rem & 127;
  const int nc = NU - s * KT_KL < KT_KL ? NU - s * KT_KL : KT_KL;
  const int r = idx & 7, hc = idx >> 3, h = hc / nc, c = hc - h * nc;
  const uint4 w = codes[q];
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
  int8_t* dst = W8 + (rg * KT_RG + r) * (long long)C + (s * KT_KL + c) * 128 + h * 64;
#pragma unroll
  for(int j = 0; j < 4; ++j){
    uint4 o;
    o.x = __builtin_amdgcn_perm(0x000100FFu, 0x000100FFu, ww[j] & 0x03030303u);
    o.y = __builtin_amdgcn_perm(0x000100FFu, 0x000100FFu, (ww[j] >> 2) & 0x03030303u);
    o.z = __builtin_amdgcn_perm(0x000100FFu, 0x000100FFu, (ww[j] >> 4) & 0x03030303u);
    o.w = __builtin_amdgcn_perm(0x000100FFu, 0x000100FFu, (ww[j] >> 6) & 0x03030303u);
    *(uint4*)(dst + 16 * j) = o;
  }
}

/* ------------------------------------------------------------------ the product */
/* a buffer resource as the 4 dwords the asm takes: base, stride 0, num_records bytes, gfx950 default flags */
__device__ __forceinline__ kt8_v4i p8_rsrc(const void* p, uint32_t bytes){
  const unsigned long long a = (unsigned long long)p;
  kt8_v4i r;
  r.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r.y = __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32) & 0xFFFF);
  r.z = (int)bytes;
  r.w = 0x00020000;
  return r;
}
/* DMA: lane i's 16 bytes at byte voff of the buffer land at LDS byte address lds + 16 i (lds wave-uniform); an offset
   past the buffer lands zeros */
__device__ __forceinline__ void p8_dma(kt8_v4i rs, uint32_t voff, uint32_t lds){
  const uint32_t l = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :: "s"(l), "v"(voff), "s"(rs) : "memory", "m0");
}
__device__ __forceinline__ uint32_t p8_lds(const void* p){
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)(const KT_L3 void*)p);
}

template <bool DBG>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2)))
k_tern_gemm8(const int8_t* __restrict__ W8, const uint16_t* __restrict__ scales, int R, int C, const int8_t* __restrict__ XQ,
             int ldq, const float* __restrict__ XS, int M, float* __restrict__ Y, uint16_t* __restrict__ Y16, int ldy,
             int32_t* __restrict__ dbg, int gx, int gy){
  extern __shared__ __attribute__((aligned(16))) uint8_t p8_lds_buf[];
  const int NG = C >> 7, R8 = kt_r8(R), ntiles = gx * gy;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), wt = w & 1, wr = w >> 1;
  const uint32_t OOB = 0x80000000u;
  const kt8_v4i rx = p8_rsrc(XQ, (uint32_t)M * (uint32_t)ldq);
  const kt8_v4i rw = p8_rsrc(W8, (uint32_t)R8 * 8u * (uint32_t)C);
  const kt8_v4i rh = p8_rsrc(scales, (uint32_t)R8 * (uint32_t)NG * 16u);
  const uint32_t lbase = p8_lds(p8_lds_buf);
  /* DMA instruction i of a wave takes rows 8 i + lane / 8 (+ 16 w activations, + 32 w trits) of the tile, chunk
     (lane % 8) ^ ((row >> 1) & 7) = (lane % 8) ^ ((lane / 8) >> 1) ^ 4 (i & 1): one source offset for the rows of even
     i and one for odd i. Rows past M or past the padded rows read past their buffer (zeros: row * stride is at least
     its size). Scales: lanes 0..3, row group 4 w + lane of the tile */
  const int pc = lane & 7, lr8 = lane >> 3;
  const uint32_t c0 = (uint32_t)((pc ^ (lr8 >> 1)) * 16), c1 = (uint32_t)((pc ^ (lr8 >> 1) ^ 4) * 16);
  /* LDS byte offsets (within a stage) of this lane's operand rows for k-chunk c: row * 128 + (c ^ ((row >> 1) & 7)) 16.
     Rows 32 i + .. of one wave share (row >> 1) & 7 = ((lane & 31) >> 1) & 7, and the k-step ks reads chunk
     2 ks + lane / 32, so the chunk part is (2 ks ^ sw) 16 with sw = that swizzle ^ lane / 32: one offset a k-step for
     the activation rows (ar0 + 32 i: + 4096 i) and one for the trit rows */
  const int ar0 = wt * 64 + (lane & 31), br0 = wr * 64 + (lane & 31);
  const int swz = (((lane & 31) >> 1) & 7) ^ (lane >> 5);
  int aoff[4], boff[4];
#pragma unroll
  for(int ks = 0; ks < 4; ++ks){
    aoff[ks] = ar0 * 128 + (((2 * ks) ^ swz) << 4);
    boff[ks] = P8_A + br0 * 128 + (((2 * ks) ^ swz) << 4);
  }

  /* the tile's sources: set by tile_at */
  int r0 = 0, n0 = 0;
  uint32_t xo[2], wo[2], so;
  auto tile_at = [&](int t){
    int bx, by;
    kt_xcd_tile(t, gx, gy, bx, by);
    r0 = bx * P8_BR; n0 = by * P8_BT;
    const uint32_t xrow = (uint32_t)(n0 + 16 * w + lr8) * (uint32_t)ldq;
    const uint32_t wrow = (uint32_t)(r0 + 32 * w + lr8) * (uint32_t)C;
    xo[0] = xrow + c0; xo[1] = xrow + c1;
    wo[0] = wrow + c0; wo[1] = wrow + c1;
    const int srg = (r0 >> 3) + 4 * w + lane;
    so = lane < 4 && srg < R8 ? (uint32_t)srg * (uint32_t)NG * 16u : OOB;
  };
  /* the DMAs of group g into stage g % 3: 7 instructions a wave */
  auto issue = [&](int g){
    const uint32_t st = lbase + (uint32_t)((g % P8_NS) * P8_STAGE);
#pragma unroll
    for(int i = 0; i < 2; ++i) p8_dma(rx, xo[i & 1] + (uint32_t)(8 * i * ldq + g * 128), st + (16 * w + 8 * i) * 128);
#pragma unroll
    for(int i = 0; i < 4; ++i) p8_dma(rw, wo[i & 1] + (uint32_t)(8 * i * C + g * 128), st + P8_A + (32 * w + 8 * i) * 128);
    if(lane < 4) p8_dma(rh, so + (uint32_t)g * 16u, st + P8_A + P8_W + 64 * w);
  };
  /* the top of group g: this wave's DMAs of group g have landed when at most group g + 1's are in flight (loads retire
     in order, so the pending ones are the last issued; stores issued before them do not matter); after the barrier
     every wave's group g is in LDS and stage (g + 2) % 3 (group g - 1's) is no longer read, so group g + 2's DMAs go
     there */
  auto top = [&](int g){
    if(DBG || g + 1 >= NG) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(%0)" :: "n"(P8_DMA) : "memory");
    __syncthreads();
    if(g + 2 < NG) issue(g + 2);
  };
  /* group g's 16 MFMAs from stage g % 3 into c (from zero) and its two row scales (read now: the stage is refilled two
     groups on). The stage offset is wave-uniform: one VALU add a k-step and operand forms each read address */
  auto mma = [&](int g, kt8_v16i (&c)[2][2], uint16_t& h0, uint16_t& h1){
    const int sto = __builtin_amdgcn_readfirstlane((g % P8_NS) * P8_STAGE);
    const uint16_t* sh = (const uint16_t*)(p8_lds_buf + sto + P8_A + P8_W);
#pragma unroll
    for(int i = 0; i < 2; ++i)
#pragma unroll
      for(int j = 0; j < 2; ++j)
#pragma unroll
        for(int e = 0; e < 16; ++e) c[i][j][e] = 0;
    /* the operands of k-step ks + 1 are read while ks's MFMAs run */
    kt8_v4i A[2][2], B[2][2];
    {
      const uint8_t* pa = p8_lds_buf + (aoff[0] + sto);
      const uint8_t* pb = p8_lds_buf + (boff[0] + sto);
#pragma unroll
      for(int i = 0; i < 2; ++i){ A[0][i] = *(const kt8_v4i*)(pa + 4096 * i); B[0][i] = *(const kt8_v4i*)(pb + 4096 * i); }
    }
#pragma unroll
    for(int ks = 0; ks < 4; ++ks){
      const int cur = ks & 1;
      if(ks < 3){
        const uint8_t* pa = p8_lds_buf + (aoff[ks + 1] + sto);
        const uint8_t* pb = p8_lds_buf + (boff[ks + 1] + sto);
#pragma unroll
        for(int i = 0; i < 2; ++i){
          A[cur ^ 1][i] = *(const kt8_v4i*)(pa + 4096 * i);
          B[cur ^ 1][i] = *(const kt8_v4i*)(pb + 4096 * i);
        }
      }
#pragma unroll
      for(int i = 0; i < 2; ++i)
#pragma unroll
        for(int j = 0; j < 2; ++j) c[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[cur][i], B[cur][j], c[i][j], 0, 0, 0);
    }
    h0 = sh[br0];
    h1 = sh[br0 + 32];
  };
  float acc[2][2][16];
  /* group g's epilogue: acc += (float)v * d, in group order */
  auto epi = [&](int g, const kt8_v16i (&c)[2][2], uint16_t h0, uint16_t h1){
    const float d0 = kt_h2f(h0), d1 = kt_h2f(h1);
    const int cr0 = r0 + br0, cr1 = cr0 + 32;
#pragma unroll
    for(int i = 0; i < 2; ++i)
#pragma unroll
      for(int e = 0; e < 16; ++e){
        acc[i][0][e] = fmaf((float)c[i][0][e], d0, acc[i][0][e]);
        acc[i][1][e] = fmaf((float)c[i][1][e], d1, acc[i][1][e]);
        if(DBG){
          const int t = n0 + wt * 64 + i * 32 + (e & 3) + 8 * (e >> 2) + 4 * (lane >> 5);
          if(t < M){
            if(cr0 < R) dbg[((long long)t * R + cr0) * NG + g] = c[i][0][e];
            if(cr1 < R) dbg[((long long)t * R + cr1) * NG + g] = c[i][1][e];
          }
        }
      }
  };

  /* one pipelined step: group gm's MFMAs into cn (scales hn0/hn1) and group ge's epilogue from co (ho0/ho1), written
     out in issue order: each MFMA is followed by 4 elements of the epilogue (8 VALU operations, which run while the
     MFMA occupies the matrix pipe), and each k-step's operand reads are issued one k-step ahead. The scheduling
     barriers keep that order (the compiler would otherwise put the whole epilogue before the MFMAs) */
  auto fused = [&](int gm, kt8_v16i (&cn)[2][2], uint16_t& hn0, uint16_t& hn1, int ge, const kt8_v16i (&co)[2][2],
                   uint16_t ho0, uint16_t ho1){
    const int sto = __builtin_amdgcn_readfirstlane((gm % P8_NS) * P8_STAGE);
    const uint16_t* sh = (const uint16_t*)(p8_lds_buf + sto + P8_A + P8_W);
    const float d0 = kt_h2f(ho0), d1 = kt_h2f(ho1);
    const int cr0 = r0 + br0, cr1 = cr0 + 32;
    kt8_v4i A[2][2], B[2][2];
    {
      const uint8_t* pa = p8_lds_buf + (aoff[0] + sto);
      const uint8_t* pb = p8_lds_buf + (boff[0] + sto);
#pragma unroll
      for(int i = 0; i < 2; ++i){ A[0][i] = *(const kt8_v4i*)(pa + 4096 * i); B[0][i] = *(const kt8_v4i*)(pb + 4096 * i); }
    }
#pragma unroll
    for(int ks = 0; ks < 4; ++ks){
      const int cur = ks & 1;
      if(ks < 3){
        const uint8_t* pa = p8_lds_buf + (aoff[ks + 1] + sto);
        const uint8_t* pb = p8_lds_buf + (boff[ks + 1] + sto);
#pragma unroll
        for(int i = 0; i < 2; ++i){
          A[cur ^ 1][i] = *(const kt8_v4i*)(pa + 4096 * i);
          B[cur ^ 1][i] = *(const kt8_v4i*)(pb + 4096 * i);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for(int m = 0; m < 4; ++m){
        const int i = m >> 1, j = m & 1;
        if(ks == 0) cn[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[cur][i], B[cur][j], kt8_v16i{}, 0, 0, 0);
        else cn[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[cur][i], B[cur][j], cn[i][j], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        /* epilogue chunk ks * 4 + m: tile (ks >> 1, ks & 1) of co, elements 4 m .. 4 m + 3 */
        const int ti = ks >> 1, tj = ks & 1;
#pragma unroll
        for(int e = 4 * m; e < 4 * m + 4; ++e){
          acc[ti][tj][e] = fmaf((float)co[ti][tj][e], tj ? d1 : d0, acc[ti][tj][e]);
          if(DBG){
            const int t = n0 + wt * 64 + ti * 32 + (e & 3) + 8 * (e >> 2) + 4 * (lane >> 5);
            const int cr = tj ? cr1 : cr0;
            if(t < M && cr < R) dbg[((long long)t * R + cr) * NG + ge] = co[ti][tj][e];
          }
        }
        /* the chunk's results are taken here (an empty asm), so the compiler cannot sink the chunk to a later step */
        asm volatile("" : "+v"(acc[ti][tj][4 * m]), "+v"(acc[ti][tj][4 * m + 1]), "+v"(acc[ti][tj][4 * m + 2]),
                     "+v"(acc[ti][tj][4 * m + 3]));
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    hn0 = sh[br0];
    hn1 = sh[br0 + 32];
  };

  /* the block's tiles t, t + gridDim.x, ... (one block a CU): the next tile's first two groups are issued right after
     this tile's stores, so the store drain and the next tile's first loads overlap */
  int t = blockIdx.x;
  tile_at(t);
  issue(0);
  if(NG > 1) issue(1);
  for(; t < ntiles; ){
#pragma unroll
    for(int i = 0; i < 2; ++i)
#pragma unroll
      for(int j = 0; j < 2; ++j)
#pragma unroll
        for(int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
    /* software pipeline: group g's MFMAs are issued before group g - 1's epilogue, so the matrix cores run one group
       while the VALU scales the other (int32 set g % 2; two groups a turn of the loop keep the sets static) */
    kt8_v16i cx[2][2], cy[2][2];
    uint16_t hx0, hx1, hy0, hy1;
    top(0);
    mma(0, cx, hx0, hx1);
    int g = 1;
    for(; g + 2 <= NG; g += 2){
      top(g);
      fused(g, cy, hy0, hy1, g - 1, cx, hx0, hx1);
      top(g + 1);
      fused(g + 1, cx, hx0, hx1, g, cy, hy0, hy1);
    }
    if(g < NG){
      top(g);
      mma(g, cy, hy0, hy1);
      epi(g - 1, cx, hx0, hx1);
      epi(g, cy, hy0, hy1);
    } else epi(g - 1, cx, hx0, hx1);
    __syncthreads();                    /* every wave is done with every stage of this tile */
    /* Y = XS[t] * acc, each output through LDS: a wave stages its 64 tokens x 64 rows (the stages are free until the
       next tile's first DMAs), token rows at a 16-byte-padded pitch, then writes 16 bytes a lane, whole token rows of
       the block in contiguous runs (fp16: 8 store instructions a wave and tile in place of 64 two-byte ones). The
       launcher routes outputs not 16-byte aligned, or with ldy not a multiple of 8, to the packed-trit kernel. */
    const int tw0 = n0 + wt * 64, rw0 = r0 + wr * 64;
    auto staged = [&](auto tag, auto* Yp){
      using T = decltype(tag);
      /* the lane index taken through an empty asm: what is computed from it here is not hoisted out of the tile loop
         (where it would hold registers the products need) */
      int lane = threadIdx.x & 63;
      asm volatile("" : "+v"(lane));
      constexpr int ES = (int)sizeof(T), PITCH = 64 * ES + 16, CPR = 64 * ES / 16, TPI = 64 / CPR, EPC = 16 / ES;
      uint8_t* ob = p8_lds_buf + (size_t)w * 64 * PITCH;
      /* the wave's 64 token scales: one load a lane, through LDS (past the 8 staging blocks) to every lane */
      float* xsw = (float*)(p8_lds_buf + (size_t)8 * 64 * PITCH) + 64 * w;
      xsw[lane] = tw0 + lane < M ? XS[(long long)(tw0 + lane) * NG] : 0.0f;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for(int i = 0; i < 2; ++i)
#pragma unroll
        for(int e = 0; e < 16; ++e){
          const int lt = i * 32 + (e & 3) + 8 * (e >> 2) + 4 * (lane >> 5);
          const float xr = xsw[lt];
#pragma unroll
          for(int j = 0; j < 2; ++j){
            float y = acc[i][j][e] * xr;
            /* the fp32 product, then fp16 (two roundings, as the other products): the empty asm keeps the compiler
               from folding the multiply into a mixed-precision instruction that rounds once */
            asm volatile("" : "+v"(y));
            T* d = (T*)(ob + lt * PITCH + ((lane & 31) + 32 * j) * ES);
            if constexpr(ES == 4) *d = y;
            else *d = __half_as_ushort(__float2half_rn(y));
          }
        }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for(int k = 0; k < 64 / TPI; ++k){
        const int lt = lane / CPR + TPI * k, ck = lane % CPR, tk = tw0 + lt, row = rw0 + ck * EPC;
        if(tk < M && row < R){
          const uint4 v = *(const uint4*)(ob + lt * PITCH + ck * 16);
          T* dst = Yp + (long long)tk * ldy + row;
          if(row + EPC <= R) *(uint4*)dst = v;
          else {                                                   /* the last rows of a ragged R */
            const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for(int q = 0; q < EPC; ++q)
              if(row + q < R){
                if constexpr(ES == 4) dst[q] = __uint_as_float(vw[q]);
                else dst[q] = (uint16_t)(vw[q >> 1] >> (16 * (q & 1)));
              }
          }
        }
      }
    };
    if(Y){ staged(0.0f, Y); __syncthreads(); }
    if(Y16){ staged((uint16_t)0, Y16); __syncthreads(); }
    t += gridDim.x;
    if(t < ntiles){
      tile_at(t);
      issue(0);
      if(NG > 1) issue(1);
    }
  }
}

template __global__ void k_tern_gemm8<false>(const int8_t*, const uint16_t*, int, int, const int8_t*, int, const float*,
                                             int, float*, uint16_t*, int, int32_t*, int, int);
template __global__ void k_tern_gemm8<true>(const int8_t*, const uint16_t*, int, int, const int8_t*, int, const float*,
                                            int, float*, uint16_t*, int, int32_t*, int, int);

size_t kt_gemm8_lds(){ return (size_t)P8_NS * P8_STAGE; }
