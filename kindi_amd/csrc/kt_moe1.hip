/* kt_moe1.hip - a q8_0 MoE feed-forward for one token in two launches (kt_moe_decode at M = 1): Kindi's Lightning
   decode chain lt_router_topk (lightning.cu:414-468) -> lt_quant (70-88) -> lt_mv_q2 up (154-195) -> lt_quant2 (470)
   -> lt_mv_q2_down (197-256) -> lt_moe_combine (1352-1361).

   Both kernels compute exactly the decode product's numbers (kt_gemv.h): a matrix's K units are cut into KS slices of
   whole steps (KS a function of C only), lane 8 c + r chains fmaf((float)v, d_w * d_x, .) over its units 8 s + c of a
   slice, the 8 lanes of a row are added by the xor butterfly and the slice sums left to right; the int8 activations
   are kt_q8_quant's (relu^2 first for the down input), made per 32-column unit in the staging. Only the assignment of
   slices to waves differs, which does not change any sum. So u, yd and x have the bits of the separate launches
   (kt_moe_route + kt_q8_quant + kt_q8_grouped + kt_q8_quant(act 1) + kt_q8_grouped + kt_moe_combine).

   k_moe1_up    grid (row groups of F, k picks), ceil(KS / 2) waves: wave w computes slices w and w + ceil(KS / 2) of
                its row group of pick blockIdx.y's up matrix (two slices a wave keep the whole grid resident at once at
                the 30B-class shape). Wave 0 first computes the token's top-k (kt_topk.h); block (0, 0) writes ids,
                gw and the picks' down matrices for the next launch.
   k_moe1_down  grid (row groups of H), KS x ceil(k / 2) waves: wave (ks, g) computes slice ks of picks 2 g, 2 g + 1
                for its row group; then wave 0 adds each pick's slices in order and the picks into x in selection order,
                x[row] += sum_j fmaf(gw_j, yd_j[row], .) (+ ysh[row]). The block owns its rows, so the combine needs no
                cross-block ordering. */
#include "kt_gemv.h"
#include "kt_topk.h"

#define KM1_KMAX 8                     /* picks a token in this chain */
#define KM1_UP 48                      /* a staged 32-byte unit and its pad (LDS) */
#ifdef KT_TRACE                        /* a timeline build: per-block s_memrealtime stamps, read by kt_trace_read */
#define KT_TS(slot) do { if(threadIdx.x == 0) kt_trace_buf[(slot)] = __builtin_amdgcn_s_memrealtime(); } while(0)
extern "C" int kt_trace_read(void* host){
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(kt_trace_buf), sizeof(kt_trace_buf), 0, hipMemcpyDeviceToHost);
}
#else
#define KT_TS(slot) do {} while(0)
#endif

/* T tasks of one wave: task t is slice sl[t] of the row group rg of the kq8 matrix at base[t] against the fp32 input
   row xin[t] (quantized here, relu^2 first when RELU); y[t] = the slice sum of row 8 rg + (lane & 7), in every lane of
   the row (the butterfly's result). Every weight, scale and input load of all tasks is issued before the first use.
   on[t] = false: no task (its weight loads read task 0's addresses, its input load the row's first step; its result
   is not used). xw: T * KT_SL * 8 units
   of the wave's LDS. */
template <int T, bool RELU>
__device__ __forceinline__ void km1_tasks(const uint8_t* const (&base)[T], const int (&sl)[T],
                                          const float* const (&xin)[T], const bool (&on)[T], int R, int NU, int KS,
                                          int rg, uint8_t* xw, float (&y)[T], int lane){
  constexpr int SL = KT_SL;
  const int S = kt_steps(NU), r = lane & 7, c = lane >> 3;
  KtStep w[T][SL];
  uint4 xv[T][SL];
  int lo[T], ns[T];
#pragma unroll
  for(int t = 0; t < T; ++t){
    lo[t] = sl[t] * S / KS;
    ns[t] = (sl[t] + 1) * S / KS - lo[t];                         /* 1 or 2 steps */
    const uint4* wb = (const uint4*)base[t];
    const uint16_t* sb = (const uint16_t*)(base[t] + (long long)kt_r8(R) * NU * 256);
#pragma unroll
    for(int f = 0; f < SL; ++f){
      const int s = lo[t] + (f < ns[t] ? f : 0), u = s * KT_KL + c;
      const bool ok = on[t] && f < ns[t] && u < NU;
      const unsigned o0 = ok ? (unsigned)kt_widx(NU, rg, s, 0, c, r) : 0u;
      const unsigned o1 = ok ? (unsigned)kt_widx(NU, rg, s, 1, c, r) : 0u;
      const unsigned os = ok ? (unsigned)kt_sidx(NU, rg, u, r) : 0u;
      w[t][f].c0 = kt_ldnt(wb + o0);
      w[t][f].c1 = kt_ldnt(wb + o1);
      w[t][f].hs = sb[os];
      /* an off task (its slice may be KS, one past the row) reads step 0 of the input row: every load stays inside
         the row */
      const int sa = on[t] ? s : 0;
      const int nc = NU - sa * KT_KL < KT_KL ? NU - sa * KT_KL : KT_KL;
      const int of = lane * 4, ofc = of < nc * 32 ? of : 0;       /* unit c = lane / 8, floats 4 r .. 4 r + 3 */
      xv[t][f] = *(const uint4*)(xin[t] + (long long)sa * KT_KL * 32 + ofc);
    }
  }
  float da[T][SL];
#pragma unroll
  for(int t = 0; t < T; ++t)
#pragma unroll
    for(int f = 0; f < SL; ++f){
      const uint32_t q = kt_q8_unit_quant<RELU>(xv[t][f], da[t][f]);
      *(uint32_t*)(xw + ((t * SL + f) * KT_KL + c) * KM1_UP + 4 * r) = q;
    }
  kt_wave_sync();
#pragma unroll
  for(int t = 0; t < T; ++t){
    float acc = 0.0f;
    if(on[t]){                                                    /* uniform */
#pragma unroll
      for(int f = 0; f < SL; ++f){
        if(f < ns[t]){                                            /* uniform */
          const int u = (lo[t] + f) * KT_KL + c;
          const bool uok = u < NU;
          const float d = uok ? kt_h2f(w[t][f].hs) : 0.0f;
          int v = kt_unit_lds<KT_FMT_Q8>(w[t][f].c0, w[t][f].c1, xw + ((t * SL + f) * KT_KL + (uok ? c : 0)) * KM1_UP);
          v = uok ? v : 0;
          acc = fmaf((float)v, d * da[t][f], acc);
        }
      }
    }
    y[t] = kt_row_sum(acc);
  }
}

__global__ void __launch_bounds__(64 * KT_KSMAX / 2) __attribute__((amdgpu_waves_per_eu(4)))
k_moe1_up(const float* __restrict__ logits, int E, int k, const KtRouter rt, const uint8_t* const* __restrict__ wup,
          const uint8_t* const* __restrict__ wdown, int R, int C, const float* __restrict__ x, float* __restrict__ u,
          int* __restrict__ ids, float* __restrict__ gw, const uint8_t** __restrict__ pdown, int KS){
  __shared__ float s_gw[KM1_KMAX];
  __shared__ int s_ids[KM1_KMAX];
  __shared__ const uint8_t* s_w;
  extern __shared__ __attribute__((aligned(16))) uint8_t kt_lds[];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), r = lane & 7, c = lane >> 3;
  const int NW = (KS + 1) / 2, j = blockIdx.y, rg = blockIdx.x;
  KT_TS((j * gridDim.x + rg) * 4);
  if(wv == 0){
    /* up to 128 experts: the up table is loaded with the logits (one memory round trip before the selection) and the
       expert's pointer taken from the lane that holds it */
    const uint8_t* t0 = nullptr;
    const uint8_t* t1 = nullptr;
    if(E <= 128){
      t0 = wup[lane < E ? lane : 0];
      t1 = wup[lane + 64 < E ? lane + 64 : 0];
    }
    const int e = kt_topk_wave(logits, E, k, rt, s_ids, s_gw, lane);
    const int ej = __builtin_amdgcn_readlane(e, j);
    KT_TS((j * gridDim.x + rg) * 4 + 1);
    if(E <= 128){
      const unsigned long long a = (unsigned long long)(ej < 64 ? t0 : t1);
      const unsigned lo = __builtin_amdgcn_readlane((int)a, ej & 63), hi = __builtin_amdgcn_readlane((int)(a >> 32), ej & 63);
      if(lane == 0) s_w = (const uint8_t*)((unsigned long long)hi << 32 | lo);
    } else if(lane == 0) s_w = wup[ej];
    if(blockIdx.x == 0 && blockIdx.y == 0 && lane < k){
      ids[lane] = e;
      pdown[lane] = wdown[e];
    }
  }
  __syncthreads();
  if(threadIdx.x < k && blockIdx.x == 0 && blockIdx.y == 0) gw[threadIdx.x] = s_gw[threadIdx.x];
  const uint8_t* const b = s_w;
  const uint8_t* const bs[2] = {b, b};
  const int sl[2] = {wv, wv + NW};
  const float* const xs[2] = {x, x};
  const bool on[2] = {true, wv + NW < KS};
  float y[2];
  uint8_t* xw = kt_lds + (size_t)wv * 2 * KT_SL * KT_KL * KM1_UP;
  float* red = (float*)(kt_lds + (size_t)NW * 2 * KT_SL * KT_KL * KM1_UP);     /* [KS][8] slice sums */
  KT_TS((j * gridDim.x + rg) * 4 + 2);
  km1_tasks<2, false>(bs, sl, xs, on, R, C / 32, KS, rg, xw, y, lane);
  if(c == 0){
    red[sl[0] * 8 + r] = y[0];
    if(on[1]) red[sl[1] * 8 + r] = y[1];
  }
  __syncthreads();
  const int row = rg * KT_RG + r;
  if(wv == 0 && c == 0 && row < R) u[(long long)j * R + row] = kt_slice_sum(red + r, 8, KS);
  KT_TS((j * gridDim.x + rg) * 4 + 3);
}

__global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(2)))
k_moe1_down(const uint8_t* const* __restrict__ pdown, const float* __restrict__ gw, int k, int R, int C,
            const float* __restrict__ u, float* __restrict__ yd, float* __restrict__ x, const float* __restrict__ ysh,
            int KS){
  extern __shared__ __attribute__((aligned(16))) uint8_t kt_lds[];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), r = lane & 7, c = lane >> 3;
  const int NG = (k + 1) / 2, ks = wv % KS, g = wv / KS, rg = blockIdx.x, row = rg * KT_RG + r;
  KT_TS(32768 + rg * 4);
  /* the combine's operands first: they do not wait for anything */
  float gwv[KM1_KMAX], x0 = 0.0f, ys = 0.0f;
  if(wv == 0 && c == 0){
#pragma unroll
    for(int j = 0; j < KM1_KMAX; ++j) gwv[j] = gw[j < k ? j : 0];
    x0 = x[row < R ? row : 0];
    ys = ysh ? ysh[row < R ? row : 0] : 0.0f;
  }
  const int j0 = 2 * g, j1 = 2 * g + 1;
  const uint8_t* const bs[2] = {pdown[j0], pdown[j1 < k ? j1 : j0]};
  const int sl[2] = {ks, ks};
  const float* const xs[2] = {u + (long long)j0 * C, u + (long long)(j1 < k ? j1 : j0) * C};
  const bool on[2] = {true, j1 < k};
  float y[2];
  uint8_t* xw = kt_lds + (size_t)wv * 2 * KT_SL * KT_KL * KM1_UP;
  float* red = (float*)(kt_lds + (size_t)KS * NG * 2 * KT_SL * KT_KL * KM1_UP);   /* [KS][KMAX][8] */
  km1_tasks<2, true>(bs, sl, xs, on, R, C / 32, KS, rg, xw, y, lane);
  KT_TS(32768 + rg * 4 + 1);
  if(c == 0){
    red[(ks * KM1_KMAX + j0) * 8 + r] = y[0];
    if(on[1]) red[(ks * KM1_KMAX + j1) * 8 + r] = y[1];
  }
  __syncthreads();
  KT_TS(32768 + rg * 4 + 2);
  if(wv == 0){
    /* lane 8 j + r: pick j's row r, its slice sums in slice order; then lane r adds the picks in selection order */
    const int jj = lane >> 3;
    const float v = kt_slice_sum(red + jj * 8 + r, KM1_KMAX * 8, KS);
    if(jj < k && row < R) yd[(long long)jj * R + row] = v;
    float vj[KM1_KMAX];
#pragma unroll
    for(int q = 0; q < KM1_KMAX; ++q)
      vj[q] = __int_as_float(__builtin_amdgcn_ds_bpermute((8 * q + r) << 2, __float_as_int(v)));
    if(c == 0 && row < R){
      float s = 0.0f;
#pragma unroll
      for(int q = 0; q < KM1_KMAX; ++q) s = q < k ? fmaf(gwv[q], vj[q], s) : s;
      x[row] = x0 + (ysh ? s + ys : s);
    }
  }
  KT_TS(32768 + rg * 4 + 3);
}

size_t kt_moe1_up_lds(int KS){ return (size_t)((KS + 1) / 2) * 2 * KT_SL * KT_KL * KM1_UP + (size_t)KS * 8 * 4; }
size_t kt_moe1_down_lds(int k, int KS){
  return (size_t)KS * ((k + 1) / 2) * 2 * KT_SL * KT_KL * KM1_UP + (size_t)KS * KM1_KMAX * 8 * 4;
}
