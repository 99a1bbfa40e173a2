/* kt_moe.hip - the MoE dispatch around the q8_0 expert products (lightning.cu:348-468 router / top-k,
   1318-1349 lt_moe_lists, 1352-1361 lt_moe_combine; grouped products lt_mm_* lightning.cu:958-1168).

     k_moe_topk     softmax over E logits, the k largest, weights normalized over the chosen k. Selection compares
                    logits (the softmax is monotone, ties to the lower expert index), and the weights are
                    exp(l_j - l_max) / sum over the chosen of exp(l_i - l_max) (the full softmax denominator cancels).
     k_moe_sort     token-sorted lists: cnt / off per expert, xrow (entry -> token), where ((t, j) -> entry), and the
                    active experts in ascending order. Entries of one expert are in ascending flat index t k + j
                    (stable), so the lists are deterministic.
     k_q8_grouped   per active expert, its list's tokens against its q8_0 rows (kq8 layout), MT tokens per pass;
                    output row = list entry. Same unit arithmetic as the dense q8_0 decode product.
     k_moe_combine  x[t] += sum_j fmaf(gw[t k + j], yd[where[t k + j]], .) (+ ysh[t]).
*/
#include "kt_common.h"

extern "C" __global__ void __launch_bounds__(64) k_moe_topk(const float* __restrict__ logits, int E, int k,
                                                            int* __restrict__ ids, float* __restrict__ gw){
  /* one wave per token; E <= 1024, k <= 16 */
  const int t = blockIdx.x, lane = threadIdx.x;
  const float* l = logits + (long long)t * E;
  __shared__ int sel[16];
  __shared__ float lv[16];
  for(int j = 0; j < k; ++j){
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for(int e = lane; e < E; e += 64){
      bool used = false;
      for(int i = 0; i < j; ++i) used |= sel[i] == e;
      const float v = l[e];
      if(!used && (v > bv || (v == bv && e < bi))){ bv = v; bi = e; }
    }
#pragma unroll
    for(int o = 32; o > 0; o >>= 1){
      const float ov = __shfl_xor(bv, o);
      const int oi = __shfl_xor(bi, o);
      if(ov > bv || (ov == bv && oi < bi)){ bv = ov; bi = oi; }
    }
    if(lane == 0){ sel[j] = bi; lv[j] = bv; }
    __syncthreads();
  }
  if(lane == 0){
    float p[16], s = 0.0f;
    for(int j = 0; j < k; ++j){ p[j] = expf(lv[j] - lv[0]); s += p[j]; }
    for(int j = 0; j < k; ++j){ ids[t * k + j] = sel[j]; gw[t * k + j] = p[j] / s; }
  }
}

extern "C" __global__ void __launch_bounds__(1024) k_moe_sort(const int* __restrict__ ids, int n, int E,
    int* __restrict__ cnt, int* __restrict__ off, int* __restrict__ xrow, int* __restrict__ where,
    int* __restrict__ act, int* __restrict__ nact, int k){
  /* one block; n = M k entries. Counting with LDS atomics (order-free), a serial scan by one wave, then thread e
     walks the entries in order and places its expert's ones (stable). */
  __shared__ int c[1024], o[1024];
  __shared__ int chunk[1024];
  const int tid = threadIdx.x;
  for(int e = tid; e < E; e += 1024) c[e] = 0;
  __syncthreads();
  for(int i = tid; i < n; i += 1024) atomicAdd(&c[ids[i]], 1);
  __syncthreads();
  if(tid == 0){
    int s = 0, a = 0;
    for(int e = 0; e < E; ++e){
      o[e] = s;
      s += c[e];
      if(c[e]) act[a++] = e;
    }
    *nact = a;
  }
  __syncthreads();
  for(int e = tid; e < E; e += 1024){ cnt[e] = c[e]; off[e] = o[e]; }
  int pos = tid < E ? o[tid] : 0;
  for(int i0 = 0; i0 < n; i0 += 1024){
    __syncthreads();
    if(i0 + tid < n) chunk[tid] = ids[i0 + tid];
    __syncthreads();
    if(tid < E){
      const int m = min(1024, n - i0);
      for(int i = 0; i < m; ++i){
        if(chunk[i] == tid){
          xrow[pos] = (i0 + i) / k;
          where[i0 + i] = pos;
          ++pos;
        }
      }
    }
  }
}

/* grid (ntiles, min(E, entries)), block 256: block y = active expert y; its list's tokens in passes of MT (the
   expert's rows are re-read from L2 per pass). 4 waves take K slices of the rows, added in wave order. */
template <int MT>
__global__ void __launch_bounds__(256) k_q8_grouped(const KtGroupedArgs a){
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, tile = blockIdx.x;
  if((int)blockIdx.y >= *a.nact) return;
  const int e = a.act[blockIdx.y], ce = a.cnt[e], oe = a.off[e];
  const int row = tile * KT_TR + lane, NU = a.NU;
  const int Rp = (a.R + KT_TR - 1) / KT_TR * KT_TR;
  const uint8_t* base = a.wexp[e];
  const uint4* __restrict__ wp = (const uint4*)base + (long long)tile * NU * 128 + lane;
  const uint16_t* __restrict__ sc = (const uint16_t*)(base + (long long)Rp * a.C) + (long long)tile * NU * 64 + lane;
  const int w0 = (int)((long long)wv * NU / KT_WAVES), w1 = (int)((long long)(wv + 1) * NU / KT_WAVES);
  __shared__ float red[KT_WAVES][MT][KT_TR];

  for(int t0 = 0; t0 < ce; t0 += MT){
    const int nt = min(MT, ce - t0);
    int xr[MT];
#pragma unroll
    for(int t = 0; t < MT; ++t){
      const int p = oe + t0 + min(t, nt - 1);
      xr[t] = a.xrow ? a.xrow[p] : p;
    }
    float acc[MT];
#pragma unroll
    for(int t = 0; t < MT; ++t) acc[t] = 0.0f;
    for(int u = w0; u < w1; ++u){
      const uint4 c0 = wp[(long long)u * 128];
      const uint4 c1 = wp[(long long)u * 128 + 64];
      const float d = kt_h2f(sc[(long long)u * 64]);
      const int w[8] = {(int)c0.x, (int)c0.y, (int)c0.z, (int)c0.w, (int)c1.x, (int)c1.y, (int)c1.z, (int)c1.w};
#pragma unroll
      for(int t = 0; t < MT; ++t){
        if(t < nt){
          const int* __restrict__ x = (const int*)(a.xq + (long long)xr[t] * a.ldq) + u * 8;
          int v = 0;
#pragma unroll
          for(int j = 0; j < 8; ++j) v = kt_dot4(w[j], x[j], v);
          acc[t] = fmaf((float)v, d * a.xd[(long long)xr[t] * a.ldd + u], acc[t]);
          if(a.dbg && row < a.R) a.dbg[((long long)(oe + t0 + t) * a.R + row) * NU + u] = v;
        }
      }
    }
    __syncthreads();                                         /* the previous pass's sums are read */
#pragma unroll
    for(int t = 0; t < MT; ++t) red[wv][t][lane] = acc[t];
    __syncthreads();
    if(wv == 0 && row < a.R){
#pragma unroll
      for(int t = 0; t < MT; ++t)
        if(t < nt)
          a.y[(long long)(oe + t0 + t) * a.ldy + row] = ((red[0][t][lane] + red[1][t][lane]) + red[2][t][lane]) + red[3][t][lane];
    }
  }
}
template __global__ void k_q8_grouped<1>(const KtGroupedArgs);
template __global__ void k_q8_grouped<4>(const KtGroupedArgs);
template __global__ void k_q8_grouped<8>(const KtGroupedArgs);
template __global__ void k_q8_grouped<16>(const KtGroupedArgs);

extern "C" __global__ void __launch_bounds__(256) k_moe_combine(const float* __restrict__ yd, const float* __restrict__ ysh,
    const int* __restrict__ where, const float* __restrict__ gw, int k, int cols, float* __restrict__ x){
  const int t = blockIdx.x;
  for(int i = threadIdx.x; i < cols; i += blockDim.x){
    float s = 0.0f;
    for(int j = 0; j < k; ++j) s = fmaf(gw[t * k + j], yd[(long long)where[t * k + j] * cols + i], s);
    x[(long long)t * cols + i] += ysh ? s + ysh[(long long)t * cols + i] : s;
  }
}
