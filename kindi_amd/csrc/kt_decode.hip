/* kt_decode.hip - gfx950 kernels of the decode side of the quantized linear layer:
     k_tern_pack   reference pack (convert.py:144-159 bcodes [C/4][R], dpm [C/128][R]) -> kt2 device layout, or
                   the same bytes after Kindi's load-time GEMV repack (layout.py:14-48) -> kt2
     k_tern_pack_ptq1  GGUF PTQ1_0 rows (28-byte blocks, convert.py:33-46) -> kt2, a range of row groups a launch
     k_q8_pack     GGUF Q8_0 rows (34-byte blocks) -> kq8 device layout
     k_quant_tern  fp32 rows -> int8 per 128-column group (or per row), XS, XA   (k_tc_q8, tc_hip.cu:43-74)
     k_quant_q8    fp32 rows -> int8 per 32-column block, fp16-rounded scale   (quant_q8, dsv41_cpu.c:251-280)
   (the decode product itself, k_gemv_flat, is in kt_gemv.h) */
#include "kt_common.h"

/* ------------------------------------------------------------------ weights: layouts */
/* the (rg, u, h, r) of code word i of a matrix with NU units (the inverse of kt_widx, word j = i & 3) */
__device__ __forceinline__ void kt_word_pos(long long i, int NU, int& rg, int& u, int& h, int& r){
  const long long per_rg = (long long)NU * 64;                /* words per row group */
  rg = (int)(i / per_rg);
  const int w = (int)(i - rg * per_rg), s = w >> 9, nc = min(KT_KL, NU - s * KT_KL), k = (w & 511) >> 2;
  h = k / (nc * 8);
  const int cr = k - h * nc * 8;
  u = s * KT_KL + (cr >> 3);
  r = cr & 7;
}

/* where the reference's pack byte s (columns 4 s .. 4 s + 3) of a row, and its fp16 scale of group p, sit in a source
   buffer. KT_SRC_PACK: the pack itself, bcodes [C/4][R], dpm [C/128][R] (convert.py:144-159). KT_SRC_G4: Kindi's
   load-time GEMV layout (layout.repack, layout.py:32-48; read back the same way by k_deq_emb3, kindi.cu:525-536):
   bytes [R/16][C/512][4 chunks of 4 rows][32 lanes][4 rows][4 bytes], scales [R/16][C/512][32 lanes][2], where lane
   l of a 16-row group holds rows b(l), b(l) + 1 (b(l) = 8 (l & 1) + 4 (l >> 1 & 1) + 2 (l >> 2 & 1)) of group
   4 ph + (l >> 3). R % 16 == 0 and C % 512 == 0 there (layout.py:38-39). */
#define KT_SRC_PACK 0
#define KT_SRC_G4 1
template <int SRC>
__device__ __forceinline__ long long kt_src_byte(int s, int row, int R, int C){
  if(SRC == KT_SRC_PACK) return (long long)s * R + row;
  return ((((long long)(row >> 4) * (C >> 9) + (s >> 7)) * 4 + ((row >> 2) & 3)) * 32 + ((s >> 2) & 31)) * 16
         + (row & 3) * 4 + (s & 3);
}
template <int SRC>
__device__ __forceinline__ long long kt_src_scale(int p, int row, int R, int C){
  if(SRC == KT_SRC_PACK) return (long long)p * R + row;
  const int rr = row & 15, lane = ((p & 3) << 3) | ((rr >> 3) & 1) | (((rr >> 2) & 1) << 1) | (((rr >> 1) & 1) << 2);
  return (((long long)(row >> 4) * (C >> 9) + (p >> 2)) * 32 + lane) * 2 + (rr & 1);
}

template <int SRC>
__global__ void k_tern_pack(const uint8_t* __restrict__ bc, const uint16_t* __restrict__ dpm, int R, int C,
                            uint32_t* __restrict__ codes, uint16_t* __restrict__ scales){
  /* one thread per output word */
  const int NG = C >> 7, R8 = kt_r8(R);
  const long long nw = (long long)R8 * NG * 64;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if(i < nw){
    int rg, u, h, r;
    kt_word_pos(i, NG, rg, u, h, r);
    const int j = (int)(i & 3), row = rg * KT_RG + r;
    uint32_t w = 0x55555555u;                                  /* padding rows: digit 1 (weight 0) everywhere */
    if(row < R){
      w = 0u;
      const int s0 = (u * 128 + h * 64 + j * 16) >> 2;        /* 4 pack bytes: columns 4k .. 4k+3 of the word */
#pragma unroll
      for(int k = 0; k < 4; ++k){
        unsigned int b = bc[kt_src_byte<SRC>(s0 + k, row, R, C)];
#pragma unroll
        for(int e = 0; e < 4; ++e){                            /* column 4k + e: byte e, bits 2k */
          w |= (b % 3u) << (8 * e + 2 * k);
          b /= 3u;
        }
      }
    }
    codes[i] = w;
  }
  const long long ns = (long long)R8 * NG * 8;
  if(i < ns){
    const int r = (int)(i & 7), u = (int)((i >> 3) % NG), rg = (int)((i >> 3) / NG), row = rg * KT_RG + r;
    scales[i] = row < R ? dpm[kt_src_scale<SRC>(u, row, R, C)] : (uint16_t)0;
  }
}
template __global__ void k_tern_pack<KT_SRC_PACK>(const uint8_t*, const uint16_t*, int, int, uint32_t*, uint16_t*);
template __global__ void k_tern_pack<KT_SRC_G4>(const uint8_t*, const uint16_t*, int, int, uint32_t*, uint16_t*);

/* digit e (0..127) of a GGUF PTQ1_0 block (convert.py:33-46): qs bytes 0..15 hold elements n 16 + j, 16..23 hold
   80 + n 8 + j, qh bytes 24..25 hold 120 + n 2 + j; digit n of byte v = ((v 3^n) mod 256) 3 / 256 */
__device__ __forceinline__ uint32_t kt_ptq1_digit(const uint8_t* __restrict__ blk, int e){
  int byte, n;
  if(e < 80){ byte = e & 15; n = e >> 4; }
  else if(e < 120){ byte = 16 + ((e - 80) & 7); n = (e - 80) >> 3; }
  else { byte = 24 + ((e - 120) & 1); n = (e - 120) >> 1; }
  const uint32_t p3 = n == 0 ? 1u : n == 1 ? 3u : n == 2 ? 9u : n == 3 ? 27u : 81u;
  return (((uint32_t)blk[byte] * p3) & 255u) * 3u >> 8;
}

extern "C" __global__ void k_tern_pack_ptq1(const uint8_t* __restrict__ raw, int R, int C, int row0, int nrg,
                                            uint32_t* __restrict__ codes, uint16_t* __restrict__ scales){
  /* one thread per output word of row groups row0 / 8 .. + nrg; raw = the GGUF rows from row0 on (C / 128 blocks of
     28 bytes a row) */
  const int NG = C >> 7, rg0 = row0 >> 3;
  const long long nw = (long long)nrg * NG * 64;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if(i < nw){
    int rg, u, h, r;
    kt_word_pos(i, NG, rg, u, h, r);
    const int j = (int)(i & 3), row = (rg0 + rg) * KT_RG + r;
    uint32_t w = 0x55555555u;                                  /* padding rows: digit 1 (weight 0) everywhere */
    if(row < R){
      w = 0u;
      const uint8_t* blk = raw + ((long long)(row - row0) * NG + u) * 28;
      const int e0 = h * 64 + j * 16;
#pragma unroll
      for(int m = 0; m < 16; ++m) w |= kt_ptq1_digit(blk, e0 + m) << (8 * (m & 3) + 2 * (m >> 2));
    }
    codes[(long long)rg0 * NG * 64 + i] = w;
  }
  const long long ns = (long long)nrg * NG * 8;
  if(i < ns){
    const int r = (int)(i & 7), u = (int)((i >> 3) % NG), rg = (int)((i >> 3) / NG), row = (rg0 + rg) * KT_RG + r;
    uint16_t v = 0;
    if(row < R){
      const uint8_t* blk = raw + ((long long)(row - row0) * NG + u) * 28;
      v = (uint16_t)(blk[26] | (blk[27] << 8));
    }
    scales[(long long)rg0 * NG * 8 + i] = v;
  }
}

extern "C" __global__ void k_q8_pack(const uint8_t* __restrict__ rows, int R, int C, uint32_t* __restrict__ codes,
                                     uint16_t* __restrict__ scales){
  /* one thread per output word; word j of half h = codes 16 h + 4 j .. +3 of block u */
  const int NB = C >> 5, R8 = kt_r8(R);
  const long long nw = (long long)R8 * NB * 64;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if(i < nw){
    int rg, u, h, r;
    kt_word_pos(i, NB, rg, u, h, r);
    const int j = (int)(i & 3), row = rg * KT_RG + r;
    uint32_t w = 0u;
    if(row < R){
      const uint8_t* p = rows + ((long long)row * NB + u) * 34 + 2 + h * 16 + j * 4;
      w = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
    }
    codes[i] = w;
  }
  const long long ns = (long long)R8 * NB * 8;
  if(i < ns){
    const int r = (int)(i & 7), u = (int)((i >> 3) % NB), rg = (int)((i >> 3) / NB), row = rg * KT_RG + r;
    uint16_t v = 0;
    if(row < R){
      const uint8_t* p = rows + ((long long)row * NB + u) * 34;
      v = (uint16_t)(p[0] | (p[1] << 8));
    }
    scales[i] = v;
  }
}

/* ------------------------------------------------------------------ activations */
__device__ __forceinline__ float kt_wave_max(float v){
#pragma unroll
  for(int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ int kt_wave_sum(int v){
#pragma unroll
  for(int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

/* grid (M), block 256: one token row. Each wave takes groups w, w + 4, ...; a lane holds columns 2l, 2l+1 of the
   group. per_row 1: amax over the whole row first (the same formula with one scale per row). per_row 2 (hp, k_tc_q8
   with hp, tc.cu:195-209): two rows a token, 2n the group's int8 row as per_row 0, 2n + 1 its residual
   r = v - q (amax / 127) (one fma, as the reference's compiler contracts it) quantized with the fixed amax
   a2 = amax / 254: q2 = clamp(rne(r (127 / a2)), -127, 127), XS = a2 / 127, XA = sum q2 (tcq128 tc.cu:160-194). */
extern "C" __global__ void __launch_bounds__(256) k_quant_tern(const float* __restrict__ X, int ldx, int C, int per_row,
                                                               int8_t* __restrict__ Q, int ldq, float* __restrict__ XS,
                                                               int* __restrict__ XA){
  const int n = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6, NG = C >> 7;
  const float* x = X + (long long)n * ldx;
  __shared__ float red[4];
  float rmax = 0.0f;
  if(per_row == 1){
    float a = 0.0f;
    for(int c = threadIdx.x * 2; c < C; c += 512){
      const float2 v = *(const float2*)(x + c);
      a = fmaxf(a, fmaxf(fabsf(v.x), fabsf(v.y)));
    }
    a = kt_wave_max(a);
    if(lane == 0) red[w] = a;
    __syncthreads();
    rmax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  }
  for(int g = w; g < NG; g += 4){
    const float2 v = *(const float2*)(x + g * 128 + 2 * lane);
    const float amax = per_row == 1 ? rmax : kt_wave_max(fmaxf(fabsf(v.x), fabsf(v.y)));
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    const int q0 = __float2int_rn(v.x * id), q1 = __float2int_rn(v.y * id);
    const int s = kt_wave_sum(q0 + q1);
    const long long n0 = per_row == 2 ? 2 * n : n;
    *(uint16_t*)(Q + n0 * ldq + g * 128 + 2 * lane) = (uint16_t)((q0 & 255) | ((q1 & 255) << 8));
    if(lane == 0){
      XS[n0 * NG + g] = amax / 127.0f;
      XA[n0 * NG + g] = s;
    }
    if(per_row == 2){                                               /* wave-uniform */
      const float sc = amax / 127.0f, a2 = amax / 254.0f, id2 = a2 != 0.0f ? 127.0f / a2 : 0.0f;
      const float r0 = fmaf(-(float)q0, sc, v.x), r1 = fmaf(-(float)q1, sc, v.y);
      const int p0 = max(-127, min(127, __float2int_rn(r0 * id2))), p1 = max(-127, min(127, __float2int_rn(r1 * id2)));
      const int s2 = kt_wave_sum(p0 + p1);
      *(uint16_t*)(Q + (n0 + 1) * ldq + g * 128 + 2 * lane) = (uint16_t)((p0 & 255) | ((p1 & 255) << 8));
      if(lane == 0){
        XS[(n0 + 1) * NG + g] = a2 / 127.0f;
        XA[(n0 + 1) * NG + g] = s2;
      }
    }
  }
}

/* grid (ceil(C/32 / 8), M), block 256: a group of 32 lanes quantizes one 32-column block (llama.cpp's CPU q8_0
   rounding: d = fp16(amax / 127), q = rne(x * 127 / amax)). act = 1: relu^2 is applied to x first (the MoE
   intermediate, lightning.cu lt_quant2). */
extern "C" __global__ void __launch_bounds__(256) k_quant_q8(const float* __restrict__ X, int ldx, int C, int act,
                                                             int8_t* __restrict__ Q, int ldq, float* __restrict__ D, int ldd){
  /* a thread takes 4 consecutive columns (one 16-byte load, one 4-byte store), 8 lanes a 32-column block, 32 blocks a
     256-thread block; the block's absmax by 3 VALU lane exchanges (max is exact in any order) */
  const int n = blockIdx.y, b = blockIdx.x * 32 + (threadIdx.x >> 3), l = threadIdx.x & 7;
  const bool ok = b * 32 < C;                                 /* whole 8-lane groups leave together */
  const int bb = ok ? b : 0;
  const float4 x = *(const float4*)(X + (long long)n * ldx + bb * 32 + 4 * l);
  float v[4] = {x.x, x.y, x.z, x.w};
  float a = 0.0f;
#pragma unroll
  for(int i = 0; i < 4; ++i){
    if(act){ v[i] = fmaxf(v[i], 0.0f); v[i] = v[i] * v[i]; }
    a = fmaxf(a, fabsf(v[i]));
  }
  a = fmaxf(a, kf_xorf<1>(a));
  a = fmaxf(a, kf_xorf<2>(a));
  a = fmaxf(a, kf_xorf<4>(a));
  const float id = a != 0.0f ? 127.0f / a : 0.0f;
  uint32_t q = 0;
#pragma unroll
  for(int i = 0; i < 4; ++i) q |= (uint32_t)(uint8_t)(int8_t)__float2int_rn(v[i] * id) << (8 * i);
  if(ok){
    *(uint32_t*)(Q + (long long)n * ldq + b * 32 + 4 * l) = q;
    if(l == 0) D[(long long)n * ldd + b] = __half2float(__float2half_rn(a / 127.0f));
  }
}

/* ------------------------------------------------------------------ the split parts of a k_tc_mv launch */
/* the part sums of a split product (k_tc_sum, tc_hip.cu:271-279): y[n R + r] = P_0 + P_1 + ... + P_{sp-1} in part
   order, P_p = P[(n sp + p) R + r]. Grid (row blocks, tokens): thread r of token blockIdx.y; the parts are read 8 at a
   time with every load of a batch issued before the first add, then added left to right. */
extern "C" __global__ void __launch_bounds__(256) k_tern_sum(const float* __restrict__ P, float* __restrict__ y, int R,
                                                             int ntok, int sp){
  (void)ntok;
  const int r = blockIdx.x * 256 + threadIdx.x;
  if(r >= R) return;
  const long long n = blockIdx.y;
  const float* col = P + n * sp * R + r;
  float acc = col[0];
  for(int p0 = 1; p0 < sp; p0 += 8){
    float v[8];
#pragma unroll
    for(int k = 0; k < 8; ++k) v[k] = p0 + k < sp ? col[(long long)(p0 + k) * R] : 0.0f;
#pragma unroll
    for(int k = 0; k < 8; ++k) if(p0 + k < sp) acc += v[k];
  }
  y[n * R + r] = acc;
}
