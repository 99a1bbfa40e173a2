/* kt_decode.hip - gfx950 kernels of the decode side of the quantized linear layer:
     k_tern_pack   reference pack (convert.py:144-159 bcodes [C/4][R], dpm [C/128][R]) -> kt2 device layout
     k_q8_pack     GGUF Q8_0 rows (34-byte blocks) -> kq8 device layout
     k_quant_tern  fp32 rows -> int8 per 128-column group (or per row), XS, XA   (k_tc_q8, tc_hip.cu:43-74)
     k_quant_q8    fp32 rows -> int8 per 32-column block, fp16-rounded scale   (quant_q8, dsv41_cpu.c:251-280)
     k_gemv<FMT,MT> the wave64 bandwidth product for 1 .. 16 tokens, ternary or q8_0 (k_tc_mv*, tc_hip.cu:180-240;
                    lt_mv_q8, lightning.cu:258-284)

   The product kernel: one lane per weight row, 64 rows per wave, each lane streaming its row's 32-byte units with
   two 128-bit loads (a wave's loads are 1 KB contiguous). The activations of a unit are the same for every lane, so
   they are read with scalar loads into SGPRs and enter v_dot4_i32_i8 as a uniform operand. Ternary digits are
   isolated with one AND per 4 columns (slots 0..2 keep their 4^s factor and are shifted back exactly after the
   unit; slot 3 takes one shift), so a unit costs 8 x (4 dot4 + 5 logic ops) per lane, independent of the trit
   values. The four waves of a block take consecutive K slices of the block's split and are added in LDS in wave
   order; splits of K across blocks are added by the last block to arrive, in split order. */
#include "kt_common.h"

/* ------------------------------------------------------------------ weights: layouts */
extern "C" __global__ void k_tern_pack(const uint8_t* __restrict__ bc, const uint16_t* __restrict__ dpm, int R, int C,
                                       int Rp, uint32_t* __restrict__ codes, uint16_t* __restrict__ scales){
  /* one thread per output word: word index ((tile NG + g) 2 + h) 64 + l) 4 + j */
  const int NG = C >> 7;
  const long long nw = (long long)Rp * NG * 8;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if(i < nw){
    const int j = (int)(i & 3), l = (int)((i >> 2) & 63), h = (int)((i >> 8) & 1);
    const long long tg = i >> 9;
    const int g = (int)(tg % NG), tile = (int)(tg / NG), r = tile * KT_TR + l;
    uint32_t w = 0x55555555u;                                  /* padding rows: digit 1 (weight 0) everywhere */
    if(r < R){
      w = 0u;
      const int s0 = (g * 128 + h * 64 + j * 16) >> 2;        /* 4 pack bytes: columns 4k .. 4k+3 of the word */
#pragma unroll
      for(int k = 0; k < 4; ++k){
        unsigned int b = bc[(long long)(s0 + k) * R + r];
#pragma unroll
        for(int e = 0; e < 4; ++e){                            /* column 4k + e: byte e, bits 2k */
          w |= (b % 3u) << (8 * e + 2 * k);
          b /= 3u;
        }
      }
    }
    codes[i] = w;
  }
  const long long ns = (long long)Rp * NG;
  if(i < ns){
    const int l = (int)(i & 63);
    const long long tg = i >> 6;
    const int g = (int)(tg % NG), tile = (int)(tg / NG), r = tile * KT_TR + l;
    scales[i] = r < R ? dpm[(long long)g * R + r] : (uint16_t)0;
  }
}

extern "C" __global__ void k_q8_pack(const uint8_t* __restrict__ rows, int R, int C, int Rp, uint32_t* __restrict__ codes,
                                     uint16_t* __restrict__ scales){
  /* one thread per output word: ((tile NB + b) 2 + h) 64 + l) 4 + j; word = codes 16h + 4j .. +3 of block b */
  const int NB = C >> 5;
  const long long nw = (long long)Rp * NB * 8;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if(i < nw){
    const int j = (int)(i & 3), l = (int)((i >> 2) & 63), h = (int)((i >> 8) & 1);
    const long long tb = i >> 9;
    const int b = (int)(tb % NB), tile = (int)(tb / NB), r = tile * KT_TR + l;
    uint32_t w = 0u;
    if(r < R){
      const uint8_t* p = rows + ((long long)r * NB + b) * 34 + 2 + h * 16 + j * 4;
      w = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
    }
    codes[i] = w;
  }
  const long long ns = (long long)Rp * NB;
  if(i < ns){
    const int l = (int)(i & 63);
    const long long tb = i >> 6;
    const int b = (int)(tb % NB), tile = (int)(tb / NB), r = tile * KT_TR + l;
    uint16_t s = 0;
    if(r < R){
      const uint8_t* p = rows + ((long long)r * NB + b) * 34;
      s = (uint16_t)(p[0] | (p[1] << 8));
    }
    scales[i] = s;
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
   group. per_row: amax over the whole row first (the same formula with one scale per row). */
extern "C" __global__ void __launch_bounds__(256) k_quant_tern(const float* __restrict__ X, int ldx, int C, int per_row,
                                                               int8_t* __restrict__ Q, int ldq, float* __restrict__ XS,
                                                               int* __restrict__ XA){
  const int n = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6, NG = C >> 7;
  const float* x = X + (long long)n * ldx;
  __shared__ float red[4];
  float rmax = 0.0f;
  if(per_row){
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
    const float amax = per_row ? rmax : kt_wave_max(fmaxf(fabsf(v.x), fabsf(v.y)));
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    const int q0 = __float2int_rn(v.x * id), q1 = __float2int_rn(v.y * id);
    const int s = kt_wave_sum(q0 + q1);
    *(uint16_t*)(Q + (long long)n * ldq + g * 128 + 2 * lane) = (uint16_t)((q0 & 255) | ((q1 & 255) << 8));
    if(lane == 0){
      XS[(long long)n * NG + g] = amax / 127.0f;
      XA[(long long)n * NG + g] = s;
    }
  }
}

/* grid (ceil(C/32 / 8), M), block 256: a group of 32 lanes quantizes one 32-column block (llama.cpp's CPU q8_0
   rounding: d = fp16(amax / 127), q = rne(x * 127 / amax)). act = 1: relu^2 is applied to x first (the MoE
   intermediate, lightning.cu lt_quant2). */
extern "C" __global__ void __launch_bounds__(256) k_quant_q8(const float* __restrict__ X, int ldx, int C, int act,
                                                             int8_t* __restrict__ Q, int ldq, float* __restrict__ D, int ldd){
  const int n = blockIdx.y, b = blockIdx.x * 8 + (threadIdx.x >> 5), l = threadIdx.x & 31;
  if(b * 32 >= C) return;                                    /* whole 32-lane halves leave together */
  float v = X[(long long)n * ldx + b * 32 + l];
  if(act){ v = fmaxf(v, 0.0f); v = v * v; }
  float a = fabsf(v);
#pragma unroll
  for(int o = 16; o > 0; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 32));
  const float id = a != 0.0f ? 127.0f / a : 0.0f;
  Q[(long long)n * ldq + b * 32 + l] = (int8_t)__float2int_rn(v * id);
  if(l == 0) D[(long long)n * ldd + b] = __half2float(__float2half_rn(a / 127.0f));
}

/* ------------------------------------------------------------------ the product */
/* the exact value of one 32-byte unit of one row against token activations x (uniform) */
template <int FMT>
__device__ __forceinline__ int kt_unit(const uint32_t m[4][8], const int* __restrict__ x){
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

/* grid (ntiles, nsplit, npass), block 256 (4 waves). MT: tokens per pass (tokens p*MT .. of blockIdx.z = p). */
template <int FMT, int MT>
__global__ void __launch_bounds__(256) k_gemv(const KtGemvArgs a, const int8_t* __restrict__ xq,
                                              const float* __restrict__ xs, const int* __restrict__ xa,
                                              int32_t* __restrict__ dbg){
  /* the wave index is uniform: read it from lane 0 so the unit loop and the activation loads stay scalar */
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), gt = blockIdx.x, sp = blockIdx.y;
  const int t0 = blockIdx.z * MT, nt = min(MT, a.M - t0);
  int mi = 0;
  if(a.nmat > 1 && gt >= a.mat[1].tile0) mi = 1;
  if(a.nmat > 2 && gt >= a.mat[2].tile0) mi = 2;
  const KtMat mat = a.mat[mi];
  const int tile = gt - mat.tile0, row = tile * KT_TR + lane;
  const int NU = a.NU;
  const int u0 = (int)((long long)sp * NU / a.nsplit), u1 = (int)((long long)(sp + 1) * NU / a.nsplit);
  const int w0 = u0 + (int)((long long)wv * (u1 - u0) / KT_WAVES), w1 = u0 + (int)((long long)(wv + 1) * (u1 - u0) / KT_WAVES);
  const uint4* __restrict__ wp = (const uint4*)mat.codes + (long long)tile * NU * 128 + lane;
  const uint16_t* __restrict__ sc = mat.scales + (long long)tile * NU * 64 + lane;
  constexpr int XW = FMT == KT_FMT_TERN ? 32 : 8;             /* activation words per unit */
  constexpr int UB = FMT == KT_FMT_TERN ? KT_UB_TERN : KT_UB_Q8; /* units whose loads are in flight together */

  float acc[MT];
#pragma unroll
  for(int t = 0; t < MT; ++t) acc[t] = 0.0f;

  for(int ub = w0; ub < w1; ub += UB){
    uint4 c0[UB], c1[UB];
    uint16_t hs[UB];
#pragma unroll
    for(int k = 0; k < UB; ++k){
      if(ub + k < w1){
        c0[k] = kt_ldnt(wp + (long long)(ub + k) * 128);
        c1[k] = kt_ldnt(wp + (long long)(ub + k) * 128 + 64);
        hs[k] = sc[(long long)(ub + k) * 64];
      }
    }
#pragma unroll
    for(int k = 0; k < UB; ++k){
      if(ub + k < w1){
        const int u = ub + k;
        const float d = kt_h2f(hs[k]);
        uint32_t m[4][8];
        kt_split_words<FMT>(c0[k], c1[k], m);
#pragma unroll
        for(int t = 0; t < MT; ++t){
          if(t < nt){
            const int n = t0 + t;
            const int* __restrict__ x = (const int*)(xq + (long long)n * a.ldq) + u * XW;
            int v = kt_unit<FMT>(m, x);
            const float s = xs[(long long)n * a.ldxs + u];
            if(FMT == KT_FMT_TERN) v -= xa[(long long)n * a.ldxs + u];
            acc[t] = fmaf((float)v, FMT == KT_FMT_TERN ? s * d : d * s, acc[t]);
            if(dbg && row < mat.R) dbg[((long long)n * mat.R + row) * NU + u] = v;
          }
        }
      }
    }
  }

  /* the block's four K slices, added in wave order */
  __shared__ float red[KT_WAVES][MT][KT_TR];
#pragma unroll
  for(int t = 0; t < MT; ++t) red[wv][t][lane] = acc[t];
  __syncthreads();
  if(wv != 0) return;
  float q[MT];
#pragma unroll
  for(int t = 0; t < MT; ++t) q[t] = ((red[0][t][lane] + red[1][t][lane]) + red[2][t][lane]) + red[3][t][lane];
  if(a.nsplit == 1){
    if(row < mat.R){
#pragma unroll
      for(int t = 0; t < MT; ++t) if(t < nt) mat.y[(long long)(t0 + t) * mat.ldy + row] = q[t];
    }
    return;
  }
  /* split K across blocks: park this part, the last block of the tile adds the parts in split order. The parts
     and the counter are accessed with agent-scope atomics (coherent across the XCDs' L2s, which an ordinary store
     is not); the fences are workgroup-scope (they only order this wave's own accesses), because an agent-scope
     fence would write back and invalidate the whole L2 of the XCD on every block. */
  const long long grow = (long long)gt * KT_TR + lane;
#pragma unroll
  for(int t = 0; t < MT; ++t)
    if(t < nt) __hip_atomic_store(a.parts + ((long long)sp * a.M + t0 + t) * a.Rtot + grow, q[t], __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);                             /* the parts' stores have completed (sc1: write-through) */
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  int* cnt = a.counters + (long long)blockIdx.z * a.ntiles + gt;
  int last = 0;
  if(lane == 0) last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == a.nsplit - 1;
  if(!__shfl(last, 0)) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  if(row < mat.R){
#pragma unroll
    for(int t = 0; t < MT; ++t){
      if(t < nt){
        float* p = a.parts + (long long)(t0 + t) * a.Rtot + grow;
        float s = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for(int k = 1; k < a.nsplit; ++k)
          s += __hip_atomic_load(p + (long long)k * a.M * a.Rtot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        mat.y[(long long)(t0 + t) * mat.ldy + row] = s;
      }
    }
  }
  if(lane == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   /* ready for the next launch */
}

#define KT_INST(FMT, MT) template __global__ void k_gemv<FMT, MT>(const KtGemvArgs, const int8_t*, const float*, const int*, int32_t*);
KT_INST(0, 1) KT_INST(0, 2) KT_INST(0, 4) KT_INST(0, 8) KT_INST(0, 16)
KT_INST(1, 1) KT_INST(1, 2) KT_INST(1, 4) KT_INST(1, 8) KT_INST(1, 16)

/* ------------------------------------------------------------------ the split parts of a k_tc_mv launch */
/* k_tc_sum (tc_hip.cu:271-279): y[n R + r] = sum_p P[(n sp + p) R + r], parts in order */
extern "C" __global__ void k_tern_sum(const float* __restrict__ P, float* __restrict__ y, int R, int ntok, int sp){
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if(i >= (long long)R * ntok) return;
  const long long n = i / R, r = i - n * R;
  const float* q = P + n * sp * R + r;
  float s = q[0];
  for(int p = 1; p < sp; ++p) s += q[(long long)p * R];
  y[i] = s;
}
