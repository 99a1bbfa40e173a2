/* kt_moe.hip - the MoE dispatch around the q8_0 expert products (lightning.cu:348-468 router / top-k,
   1318-1349 lt_moe_lists, 1352-1361 lt_moe_combine; grouped products lt_mm_* lightning.cu:958-1168).

     k_moe_topk     the router's top-k of each token (kt_topk.h): softmax over E logits (BASELINE) or Kindi's sigmoid +
                    bias scoring; the k largest, ties to the lower expert index, weights normalized over the chosen k.
     k_moe_sort     token-sorted lists: cnt / off per expert, xrow (entry -> token), where ((t, j) -> entry), and the
                    active experts in ascending order. Entries of one expert are in ascending flat index t k + j
                    (stable), so the lists are deterministic.
   (the grouped product itself, per active expert and its token list, is the decode product k_gemv_flat in its
   grouped mode, kt_gemv.h: the dense q8_0 product's lanes, arithmetic and summation tree; output row = entry)
     k_moe_route    k_moe_topk and k_moe_sort in one launch by one wave, for up to 64 entries.
     k_moe_combine  x[t] += sum_j fmaf(gw[t k + j], yd[where[t k + j]], .) (+ ysh[t]); x and ysh rows ldx apart.
*/
#include "kt_common.h"
#include "kt_topk.h"


/* exclusive prefix sum over the wave's 64 lanes (6 lane shifts through ds_bpermute); *total = the sum */
__device__ __forceinline__ int kt_wave_excl_scan(int v, int lane, int* total){
  int inc = v;
#pragma unroll
  for(int d = 1; d < 64; d <<= 1){
    const int y = __builtin_amdgcn_ds_bpermute(((lane - d) & 63) << 2, inc);
    inc += lane >= d ? y : 0;
  }
  *total = __builtin_amdgcn_readlane(inc, 63);
  return inc - v;
}

__global__ void __launch_bounds__(64) k_moe_topk(const float* __restrict__ logits, int E, int k, const KtRouter rt,
                                                int* __restrict__ ids, float* __restrict__ gw){
  /* one wave per token; E <= 1024, k <= 16 */
  const int t = blockIdx.x;
  kt_topk_wave(logits + (long long)t * E, E, k, rt, ids + t * k, gw + t * k, threadIdx.x);
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
    int* __restrict__ nact, int k, int* __restrict__ wc){
  /* one block of 1024 threads; n = M k entries, E <= 1024; wc: 16 E ints of LDS. Counting with LDS atomics
     (order-free); offsets and the active list by block scans; placement in chunks of 1024 entries, one a thread: the
     lanes of a wave holding the same expert found by ten ballots over the expert's bits (the lane's rank among them
     in lane order), each wave's count per expert in wc, an exclusive scan of those over the 16 waves per expert; an
     entry's place = its expert's offset + the earlier waves' count + its rank, so an expert's entries keep
     ascending flat index (stable) */
  __shared__ int c[1024], o[1024], wsum[16];
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
  for(int i0 = 0; i0 < n; i0 += 1024){
    for(int q = tid; q < 16 * E; q += 1024) wc[q] = 0;
    __syncthreads();
    const int i = i0 + tid;
    const bool valid = i < n;
    const int e = valid ? ids[i] : 0;
    unsigned long long eq = __ballot(valid);
#pragma unroll
    for(int b = 0; b < 10; ++b){
      const bool bit = (e >> b) & 1;
      const unsigned long long bal = __ballot(bit);
      eq &= bit ? bal : ~bal;
    }
    const int rk = __popcll(eq & ((1ull << lane) - 1ull));
    if(valid && rk == 0) wc[w * E + e] = __popcll(eq);
    __syncthreads();
    if(tid < E){
      int run = o[tid];
      for(int ww = 0; ww < 16; ++ww){ const int t = wc[ww * E + tid]; wc[ww * E + tid] = run; run += t; }
      o[tid] = run;                                              /* the next chunk continues here */
    }
    __syncthreads();
    if(valid){
      const int p = wc[w * E + e] + rk;
      xrow[p] = i / k;
      where[i] = p;
    }
    __syncthreads();                                             /* wc is cleared for the next chunk */
  }
}

extern "C" __global__ void __launch_bounds__(1024) k_moe_sort(const int* __restrict__ ids, int n, int E,
    int* __restrict__ cnt, int* __restrict__ off, int* __restrict__ xrow, int* __restrict__ where,
    int* __restrict__ act, int* __restrict__ nact, int k){
  extern __shared__ int kt_moe_wc[];                              /* 16 E */
  kt_moe_lists(ids, n, E, cnt, off, xrow, where, act, nact, k, kt_moe_wc);
}

/* the router and the lists in one launch, by one wave (n = M k <= 64 entries, E <= 1024): the top-k of each token
   leaves entry p's expert in lane p; lane l owns experts 16 l .. 16 l + 15 (counts from the n entries, read with
   readlane); offsets and the active list by prefix sums over lanes; an entry's place is its expert's offset plus the
   entries before it with the same expert (ascending flat index, as kt_moe_sort). The same outputs as
   k_moe_topk + k_moe_sort. */
__global__ void __launch_bounds__(256) k_moe_route(const float* __restrict__ logits, int M, int E, int k,
    const KtRouter rt, int* __restrict__ ids, float* __restrict__ gw, int* __restrict__ cnt, int* __restrict__ off,
    int* __restrict__ xrow, int* __restrict__ where, int* __restrict__ act, int* __restrict__ nact,
    const float* __restrict__ x, int ldx, int H, int8_t* __restrict__ Q, int ldq, float* __restrict__ D, int ldd){
  __shared__ int o[1024];
  const int lane = threadIdx.x & 63, n = M * k;
  if(threadIdx.x >= 64){
    /* waves 1..3: the tokens' int8 rows, k_quant_q8's numbers (act 0): a 32-lane half per 32-column block */
    if(!x) return;
    /* blocks h, h + 6, ... of every token, KT_RQ at a time: their loads issued together (clamped to a real block),
       then the reductions and stores, so a half-wave waits for memory once per KT_RQ blocks, not once per block */
    const int h = (threadIdx.x - 64) >> 5, l = threadIdx.x & 31, nb = H / 32;
    constexpr int KT_RQ = 8;
    for(int t = 0; t < M; ++t)
      for(int b0 = h; b0 < nb; b0 += 6 * KT_RQ){
        float v[KT_RQ];
#pragma unroll
        for(int q = 0; q < KT_RQ; ++q){
          const int b = b0 + 6 * q;
          v[q] = x[(long long)t * ldx + (b < nb ? b : h) * 32 + l];
        }
#pragma unroll
        for(int q = 0; q < KT_RQ; ++q){
          const int b = b0 + 6 * q;
          float a = fabsf(v[q]);
          a = fmaxf(a, kf_xorf<1>(a)); a = fmaxf(a, kf_xorf<2>(a)); a = fmaxf(a, kf_xorf<4>(a));
          a = fmaxf(a, kf_xorf<8>(a)); a = fmaxf(a, kf_xorf<16>(a));
          const float id = a != 0.0f ? 127.0f / a : 0.0f;
          if(b < nb){
            Q[(long long)t * ldq + b * 32 + l] = (int8_t)__float2int_rn(v[q] * id);
            if(l == 0) D[(long long)t * ldd + b] = __half2float(__float2half_rn(a / 127.0f));
          }
        }
      }
    return;
  }
  int ep = -1;                                                     /* entry lane's expert */
  for(int t = 0; t < M; ++t){
    /* entry lanes t k .. t k + k - 1 take the picks from lanes 0 .. k - 1 */
    const int mine = kt_topk_wave(logits + (long long)t * E, E, k, rt, ids + t * k, gw + t * k, lane);
    const int got = __builtin_amdgcn_ds_bpermute(((lane - t * k) & 63) << 2, mine);
    ep = lane >= t * k && lane < t * k + k ? got : ep;
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
  int tall, all;
  int base = kt_wave_excl_scan(tot, lane, &tall), abase = kt_wave_excl_scan(na, lane, &all);
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
    const int* __restrict__ where, const float* __restrict__ gw, int k, int cols, float* __restrict__ x, int ldx){
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
    x[(long long)t * ldx + i] += ysh ? s + ysh[(long long)t * ldx + i] : s;
  }
}
