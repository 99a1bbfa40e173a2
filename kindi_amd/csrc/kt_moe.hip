/* kt_moe.hip - the MoE dispatch around the q8_0 expert products (lightning.cu:348-468 router / top-k,
   1318-1349 lt_moe_lists, 1352-1361 lt_moe_combine; grouped products lt_mm_* lightning.cu:958-1168).

     k_moe_topk     softmax over E logits, the k largest, weights normalized over the chosen k. Selection compares
                    logits (the softmax is monotone, ties to the lower expert index), and the weights are
                    exp(l_j - l_max) / sum over the chosen of exp(l_i - l_max) (the full softmax denominator cancels).
     k_moe_sort     token-sorted lists: cnt / off per expert, xrow (entry -> token), where ((t, j) -> entry), and the
                    active experts in ascending order. Entries of one expert are in ascending flat index t k + j
                    (stable), so the lists are deterministic.
     k_q8_grouped   per active expert, its list's tokens against its q8_0 rows (kq8 layout), MT tokens per pass;
                    output row = list entry. The dense q8_0 decode product's lanes, arithmetic and summation tree.
     k_moe_combine  x[t] += sum_j fmaf(gw[t k + j], yd[where[t k + j]], .) (+ ysh[t]).
*/
#include "kt_common.h"

#define KT_MOE_UB 4                   /* steps whose weight loads a grouped-product wave keeps in flight */

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

/* grid (row groups, min(E, entries)), block 64: wave (rg, y) takes active expert y's 8 rows rg for its whole list,
   MT tokens a pass (the rows are re-read from L2 for each further pass). Lanes as the dense decode product
   (k_gemv): lane 8 c + r takes units c, c + 8, ... of row r; the 8 k-lanes of a row are added by the same xor
   butterfly. Output row = list entry. */
template <int MT>
__global__ void __launch_bounds__(64) k_q8_grouped(const KtGroupedArgs a, const int8_t* __restrict__ xq,
                                                   const float* __restrict__ xd, float* __restrict__ y,
                                                   int32_t* __restrict__ dbg){
  const int lane = threadIdx.x, r = lane & 7, c = lane >> 3, rg = blockIdx.x;
  if((int)blockIdx.y >= *a.nact) return;
  const int e = a.act[blockIdx.y], ce = a.cnt[e], oe = a.off[e];
  const int row = rg * KT_RG + r, NU = a.NU, S = kt_steps(NU), R8 = kt_r8(a.R);
  const uint8_t* base = a.wexp[e];
  const uint4* __restrict__ wb = (const uint4*)base;
  const uint16_t* __restrict__ sb = (const uint16_t*)(base + (long long)R8 * NU * 256);

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
    for(int s0 = 0; s0 < S; s0 += KT_MOE_UB){
      uint4 c0[KT_MOE_UB], c1[KT_MOE_UB];
      uint16_t hs[KT_MOE_UB];
#pragma unroll
      for(int k = 0; k < KT_MOE_UB; ++k){
        const int u = (s0 + k) * KT_KL + c;
        if(s0 + k < S && u < NU){
          c0[k] = wb[kt_widx(NU, rg, s0 + k, 0, c, r)];
          c1[k] = wb[kt_widx(NU, rg, s0 + k, 1, c, r)];
          hs[k] = sb[kt_sidx(NU, rg, u, r)];
        }
      }
#pragma unroll
      for(int k = 0; k < KT_MOE_UB; ++k){
        const int u = (s0 + k) * KT_KL + c;
        if(s0 + k < S && u < NU){
          const float d = kt_h2f(hs[k]);
          const int w[8] = {(int)c0[k].x, (int)c0[k].y, (int)c0[k].z, (int)c0[k].w,
                            (int)c1[k].x, (int)c1[k].y, (int)c1[k].z, (int)c1[k].w};
#pragma unroll
          for(int t = 0; t < MT; ++t){
            if(t < nt){
              const uint4* q = (const uint4*)(xq + (long long)xr[t] * a.ldq + (long long)u * 32);
              const uint4 q0 = q[0], q1 = q[1];
              int v = kt_dot4(w[0], (int)q0.x, 0);
              v = kt_dot4(w[1], (int)q0.y, v); v = kt_dot4(w[2], (int)q0.z, v); v = kt_dot4(w[3], (int)q0.w, v);
              v = kt_dot4(w[4], (int)q1.x, v); v = kt_dot4(w[5], (int)q1.y, v); v = kt_dot4(w[6], (int)q1.z, v);
              v = kt_dot4(w[7], (int)q1.w, v);
              acc[t] = fmaf((float)v, d * xd[(long long)xr[t] * a.ldd + u], acc[t]);
              if(dbg && row < a.R) dbg[((long long)(oe + t0 + t) * a.R + row) * NU + u] = v;
            }
          }
        }
      }
    }
#pragma unroll
    for(int t = 0; t < MT; ++t){
      float v = acc[t];
      v += __shfl_xor(v, 8);
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      if(c == 0 && t < nt && row < a.R) y[(long long)(oe + t0 + t) * a.ldy + row] = v;
    }
  }
}
#define KT_GINST(MT) template __global__ void k_q8_grouped<MT>(const KtGroupedArgs, const int8_t*, const float*, float*, int32_t*);
KT_GINST(1) KT_GINST(4) KT_GINST(8) KT_GINST(16)

extern "C" __global__ void __launch_bounds__(256) k_moe_combine(const float* __restrict__ yd, const float* __restrict__ ysh,
    const int* __restrict__ where, const float* __restrict__ gw, int k, int cols, float* __restrict__ x){
  const int t = blockIdx.x;
  for(int i = threadIdx.x; i < cols; i += blockDim.x){
    float s = 0.0f;
    for(int j = 0; j < k; ++j) s = fmaf(gw[t * k + j], yd[(long long)where[t * k + j] * cols + i], s);
    x[(long long)t * cols + i] += ysh ? s + ysh[(long long)t * cols + i] : s;
  }
}
