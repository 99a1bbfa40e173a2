/* kt_moe.hip - the MoE dispatch around the q8_0 expert products (lightning.cu:348-468 router / top-k,
   1318-1349 lt_moe_lists, 1352-1361 lt_moe_combine; grouped products lt_mm_* lightning.cu:958-1168).

     k_moe_topk     softmax over E logits, the k largest, weights normalized over the chosen k. Selection compares
                    logits (the softmax is monotone, ties to the lower expert index), and the weights are
                    exp(l_j - l_max) / sum over the chosen of exp(l_i - l_max) (the full softmax denominator cancels).
     k_moe_sort     token-sorted lists: cnt / off per expert, xrow (entry -> token), where ((t, j) -> entry), and the
                    active experts in ascending order. Entries of one expert are in ascending flat index t k + j
                    (stable), so the lists are deterministic.
   (the grouped product itself, per active expert and its token list, is the decode product k_gemv_flat in its
   grouped mode, kt_gemv.h: the dense q8_0 product's lanes, arithmetic and summation tree; output row = entry)
     k_moe_route    k_moe_topk and k_moe_sort in one launch by one wave, for up to 64 entries.
     k_moe_combine  x[t] += sum_j fmaf(gw[t k + j], yd[where[t k + j]], .) (+ ysh[t]).
*/
#include "kt_common.h"


/* the k largest of E <= 1024 logits by one wave, the logits in registers (lane l holds e = l + 64 i): k rounds of a
   wave arg-max (ties to the lower index, a chosen entry masked out) on the VALU exchanges; lane 0 writes ids and the
   weights exp(l_j - l_max) / sum of the chosen */
__device__ __forceinline__ void kt_topk_wave(const float* __restrict__ l, int E, int k, int* __restrict__ ids,
                                             float* __restrict__ gw, int lane, int (&sel)[16]){
  float v[16];
#pragma unroll
  for(int i = 0; i < 16; ++i){ const int e = lane + 64 * i; v[i] = e < E ? l[e] : -INFINITY; }
  unsigned used = 0u;
  float lv[16];
#pragma unroll
  for(int j = 0; j < 16; ++j){
    sel[j] = 0; lv[j] = 0.0f;
    if(j < k){
      float bv = -INFINITY;
      int bi = 0x7FFFFFFF;
#pragma unroll
      for(int i = 0; i < 16; ++i){
        const int e = lane + 64 * i;
        if(e < E && !(used >> i & 1u) && (v[i] > bv || (v[i] == bv && e < bi))){ bv = v[i]; bi = e; }
      }
#define KT_TOPK_STEP(X) { const float ov = kf_xorf<X>(bv); const int oi = kf_xor<X>(bi); \
      if(ov > bv || (ov == bv && oi < bi)){ bv = ov; bi = oi; } }
      KT_TOPK_STEP(1) KT_TOPK_STEP(2) KT_TOPK_STEP(4) KT_TOPK_STEP(8) KT_TOPK_STEP(16) KT_TOPK_STEP(32)
#undef KT_TOPK_STEP
      bi = __builtin_amdgcn_readfirstlane(bi);
      bv = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(bv)));
      if((bi & 63) == lane) used |= 1u << (bi >> 6);
      sel[j] = bi; lv[j] = bv;
    }
  }
  if(lane == 0){
    float p[16], s = 0.0f;
#pragma unroll
    for(int j = 0; j < 16; ++j) if(j < k){ p[j] = expf(lv[j] - lv[0]); s += p[j]; }
#pragma unroll
    for(int j = 0; j < 16; ++j) if(j < k){ ids[j] = sel[j]; gw[j] = p[j] / s; }
  }
}

extern "C" __global__ void __launch_bounds__(64) k_moe_topk(const float* __restrict__ logits, int E, int k,
                                                            int* __restrict__ ids, float* __restrict__ gw){
  /* one wave per token; E <= 1024, k <= 16 */
  const int t = blockIdx.x;
  int sel[16];
  kt_topk_wave(logits + (long long)t * E, E, k, ids + t * k, gw + t * k, threadIdx.x, sel);
}

/* an exclusive scan of v over the block's 1024 threads (in-wave shuffle scan, then the 16 wave totals) */
__device__ __forceinline__ int kt_block_excl_scan(int v, int* wsum){
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for(int d = 1; d < 64; d <<= 1){
    const int y = __shfl_up(x, d);
    if(lane >= d) x += y;
  }
  if(lane == 63) wsum[w] = x;
  __syncthreads();
  int pre = 0;
  for(int i = 0; i < w; ++i) pre += wsum[i];
  __syncthreads();
  return pre + x - v;
}

__device__ __forceinline__ void kt_moe_lists(const int* __restrict__ ids, int n, int E, int* __restrict__ cnt,
    int* __restrict__ off, int* __restrict__ xrow, int* __restrict__ where, int* __restrict__ act,
    int* __restrict__ nact, int k){
  /* one block of 1024 threads; n = M k entries, E <= 1024. Counting with LDS atomics (order-free); offsets and the
     active list by block scans; placement by one wave per expert (experts w, w + 16, ...): over the entries in
     order, 64 at a time, a ballot of the matches gives each its rank, so an expert's entries keep ascending flat
     index (stable) */
  __shared__ int c[1024], o[1024], wsum[16];
  __shared__ int chunk[2048];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  c[tid] = 0;
  __syncthreads();
  for(int i = tid; i < n; i += 1024) atomicAdd(&c[ids[i]], 1);
  __syncthreads();
  const int ce = tid < E ? c[tid] : 0;
  const int oe = kt_block_excl_scan(ce, wsum);
  const int ae = kt_block_excl_scan(ce > 0 ? 1 : 0, wsum);
  if(tid < E){
    o[tid] = oe;
    cnt[tid] = ce;
    off[tid] = oe;
    if(ce > 0) act[ae] = tid;
    if(tid == E - 1) *nact = ae + (ce > 0 ? 1 : 0);
  }
  __syncthreads();
  for(int i0 = 0; i0 < n; i0 += 2048){
    const int m = min(2048, n - i0);
    for(int i = tid; i < m; i += 1024) chunk[i] = ids[i0 + i];
    __syncthreads();
    for(int e = w; e < E; e += 16){
      int pos = o[e];
      for(int j = 0; j < m; j += 64){
        const bool hit = j + lane < m && chunk[j + lane] == e;
        const unsigned long long b = __ballot(hit);
        if(hit){
          const int p = pos + __popcll(b & ((1ull << lane) - 1ull));
          xrow[p] = (i0 + j + lane) / k;
          where[i0 + j + lane] = p;
        }
        pos += __popcll(b);
      }
      if(lane == 0) o[e] = pos;                                 /* the next chunk continues here */
    }
    __syncthreads();
  }
}

extern "C" __global__ void __launch_bounds__(1024) k_moe_sort(const int* __restrict__ ids, int n, int E,
    int* __restrict__ cnt, int* __restrict__ off, int* __restrict__ xrow, int* __restrict__ where,
    int* __restrict__ act, int* __restrict__ nact, int k){
  kt_moe_lists(ids, n, E, cnt, off, xrow, where, act, nact, k);
}

/* the router and the lists in one launch, by one wave (n = M k <= 64 entries, E <= 1024): the top-k of each token
   leaves entry p's expert in lane p; lane l owns experts 16 l .. 16 l + 15 (counts from the n entries, read with
   readlane); offsets and the active list by prefix sums over lanes; an entry's place is its expert's offset plus the
   entries before it with the same expert (ascending flat index, as kt_moe_sort). The same outputs as
   k_moe_topk + k_moe_sort. */
extern "C" __global__ void __launch_bounds__(256) k_moe_route(const float* __restrict__ logits, int M, int E, int k,
    int* __restrict__ ids, float* __restrict__ gw, int* __restrict__ cnt, int* __restrict__ off,
    int* __restrict__ xrow, int* __restrict__ where, int* __restrict__ act, int* __restrict__ nact,
    const float* __restrict__ x, int ldx, int H, int8_t* __restrict__ Q, int ldq, float* __restrict__ D, int ldd){
  __shared__ int o[1024];
  const int lane = threadIdx.x & 63, n = M * k;
  if(threadIdx.x >= 64){
    /* waves 1..3: the tokens' int8 rows, k_quant_q8's numbers (act 0): a 32-lane half per 32-column block */
    if(!x) return;
    const int h = (threadIdx.x - 64) >> 5, l = threadIdx.x & 31, nb = H / 32;
    for(int t = 0; t < M; ++t)
      for(int b = h; b < nb; b += 6){
        const float v = x[(long long)t * ldx + b * 32 + l];
        float a = fabsf(v);
        a = fmaxf(a, kf_xorf<1>(a)); a = fmaxf(a, kf_xorf<2>(a)); a = fmaxf(a, kf_xorf<4>(a));
        a = fmaxf(a, kf_xorf<8>(a)); a = fmaxf(a, kf_xorf<16>(a));
        const float id = a != 0.0f ? 127.0f / a : 0.0f;
        Q[(long long)t * ldq + b * 32 + l] = (int8_t)__float2int_rn(v * id);
        if(l == 0) D[(long long)t * ldd + b] = __half2float(__float2half_rn(a / 127.0f));
      }
    return;
  }
  int ep = -1;                                                     /* entry lane's expert */
  for(int t = 0; t < M; ++t){
    int sel[16];
    kt_topk_wave(logits + (long long)t * E, E, k, ids + t * k, gw + t * k, lane, sel);
#pragma unroll
    for(int j = 0; j < 16; ++j) if(j < k && lane == t * k + j) ep = sel[j];
  }
  int c[16];
#pragma unroll
  for(int i = 0; i < 16; ++i) c[i] = 0;
  for(int q = 0; q < n; ++q){
    const int d = __builtin_amdgcn_readlane(ep, q) - 16 * lane;
#pragma unroll
    for(int i = 0; i < 16; ++i) c[i] += d == i ? 1 : 0;
  }
  int tot = 0, na = 0;
#pragma unroll
  for(int i = 0; i < 16; ++i){ tot += c[i]; na += c[i] > 0 ? 1 : 0; }
  int base = 0, abase = 0, all = 0;
  for(int l = 0; l < 64; ++l){
    const int tl = __builtin_amdgcn_readlane(tot, l), al = __builtin_amdgcn_readlane(na, l);
    base += l < lane ? tl : 0;
    abase += l < lane ? al : 0;
    all += al;
  }
#pragma unroll
  for(int i = 0; i < 16; ++i){
    const int e = 16 * lane + i;
    if(e < E){
      cnt[e] = c[i];
      off[e] = base;
      o[e] = base;
      if(c[i] > 0) act[abase++] = e;
    }
    base += c[i];
  }
  if(lane == 0) *nact = all;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");        /* o[] by this wave only: a wave barrier suffices */
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  if(lane < n){
    int rank = 0;
    for(int q = 0; q < n; ++q) rank += (q < lane && __builtin_amdgcn_readlane(ep, q) == ep) ? 1 : 0;
    const int pos = o[ep] + rank;
    xrow[pos] = lane / k;
    where[lane] = pos;
  }
}

extern "C" __global__ void __launch_bounds__(256) k_moe_combine(const float* __restrict__ yd, const float* __restrict__ ysh,
    const int* __restrict__ where, const float* __restrict__ gw, int k, int cols, float* __restrict__ x){
  /* grid (column blocks of 256, tokens): one column of one token a thread, so its k loads are in flight together;
     the pairs of the token read once a block */
  __shared__ int wp[16];
  __shared__ float gp[16];
  const int t = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
  if(threadIdx.x < k){ wp[threadIdx.x] = where[t * k + threadIdx.x]; gp[threadIdx.x] = gw[t * k + threadIdx.x]; }
  __syncthreads();
  if(i < cols){
    float s = 0.0f;
    for(int j = 0; j < k; ++j) s = fmaf(gp[j], yd[(long long)wp[j] * cols + i], s);
    x[(long long)t * cols + i] += ysh ? s + ysh[(long long)t * cols + i] : s;
  }
}
