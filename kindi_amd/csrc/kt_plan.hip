/* kt_plan.hip - the decode plan executor: a sequence of ternary products (the per-layer launches of a decode step,
   spec.py:619-673: q/k/v, o, gate/up, down, ...) run by one persistent launch.

   The grid holds exactly the blocks the GPU keeps resident at once (occupancy query at build time). A block has W
   data waves (W = the largest K-slice count of the plan's stages) and one control wave:
   - stage s of the plan is cut into items of W / KS_s row groups; block b takes items b, b + G, b + 2 G, ...;
     data wave dw takes row group dw / KS_s of the item and its K slice dw % KS_s, and computes exactly what
     k_gemv_flat computes for it (the same loads, lanes, chains and butterfly), leaving the slice sum in LDS;
   - the control wave adds the KS_s slice sums of each row in slice order and stores the row, so every output bit
     equals the single-launch product's;
   - a data wave issues the weight loads of its next task (which may be in a later stage: weights never depend on
     earlier stages) before it waits for its current one, so the weight stream keeps going across stage ends;
   - stage s + 1 starts after every block has finished stage s: the control wave releases its stores (agent
     scope), arrives (a two-level count) and spins (bounded) on a flag until all G blocks have arrived, then
     acquires, and the block's data waves go on (block barrier). That is the ordering and visibility of separate stream-ordered
     launches: a stage may read anything an earlier stage wrote.
   The control wave issues no weight loads, so its fences and its spin wait for nothing but its own stores and
   atomics. The plan (header, stages) is read-only in the launch and the barrier counters and status word come as a
   separate argument, so the stage fields are scalar loads. A spin that runs out of iterations sets the plan's status word and every later barrier then passes at
   once, so a failed plan ends instead of hanging (kt_plan_status reports it). */
#include "kt_gemv.h"

#ifndef KT_SPIN_MAX
#define KT_SPIN_MAX (1u << 18)        /* spin iterations of one barrier (each at least one memory round trip) */
#endif

__device__ __forceinline__ const KtPStage& kt_stage_at(const uint8_t* plan, int s){
  return ((const KtPStage*)(plan + KT_PLAN_HDR))[s];
}

/* the grid barrier of the control wave before stage k + 1 (k = 0, 1, ...): release; arrive on the sub-counter of
   the block's group of KT_BAR_GROUP blocks; the group's last arriver arrives on the root counter, and the root's
   last arriver raises the flag to k + 1; every block spins (bounded) until the flag reaches k + 1; acquire. Counts
   only grow (targets (k + 1) x size), so one set of counters serves every stage; a block cannot arrive at barrier
   k + 1 before all have arrived at k. The counters sit on their own 128-byte lines. */
__device__ __forceinline__ void kt_plan_barrier(unsigned* ctr, unsigned k, unsigned G, int lane){
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  if(lane == 0){
    unsigned* flag = ctr + KT_BAR_FLAG * 32;
    unsigned* root = ctr + KT_BAR_ROOT * 32;
    unsigned* status = ctr + KT_BAR_STATUS * 32;
    const unsigned g = blockIdx.x / KT_BAR_GROUP, ng = (G + KT_BAR_GROUP - 1) / KT_BAR_GROUP;
    const unsigned gsize = min((unsigned)KT_BAR_GROUP, G - g * KT_BAR_GROUP);
    unsigned* sub = ctr + (KT_BAR_SUB + g) * 32;
    if(__hip_atomic_fetch_add(sub, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (k + 1) * gsize - 1u &&
       __hip_atomic_fetch_add(root, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (k + 1) * ng - 1u)
      __hip_atomic_store(flag, k + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if(__hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u){
      unsigned n = 0;
      while(__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < k + 1u){
        __builtin_amdgcn_s_sleep(1);
        if(++n == KT_SPIN_MAX){
          __hip_atomic_fetch_or(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

/* one task of a data wave: item i of stage s */
struct KtTask {
  int s, i;
};

/* (tasks are wave-uniform: readfirstlane keeps them, and the stage loads they index, scalar) */
__device__ __forceinline__ KtTask kt_first_task(const uint8_t* plan, int ns, int b){
  KtTask t = {0, b};
  while(t.s < ns && t.i >= kt_stage_at(plan, t.s).nitems){ ++t.s; t.i = b; }
  t.s = __builtin_amdgcn_readfirstlane(t.s);
  t.i = __builtin_amdgcn_readfirstlane(t.i);
  return t;
}

__device__ __forceinline__ KtTask kt_next_task(const uint8_t* plan, int ns, int b, int G, KtTask t){
  t.i += G;
  while(t.s < ns && t.i >= kt_stage_at(plan, __builtin_amdgcn_readfirstlane(t.s)).nitems){ ++t.s; t.i = b; }
  t.s = __builtin_amdgcn_readfirstlane(t.s);
  t.i = __builtin_amdgcn_readfirstlane(t.i);
  return t;
}

template <int MT>
__global__ void __launch_bounds__(1024) k_plan(const uint8_t* __restrict__ plan, unsigned* __restrict__ ctr){
  extern __shared__ __attribute__((aligned(16))) uint8_t kt_lds[];
  using F = KtFlat<KT_FMT_TERN, MT>;
  constexpr int UW = F::UW, UP = F::UP, SL = KT_SL;
  const KtPlanHdr& H = *(const KtPlanHdr*)plan;
  const int nS = H.nstages, G = H.G, W = H.W, b = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int r = lane & 7, c = lane >> 3;
  float* red = (float*)(kt_lds + (size_t)W * F::XW);             /* [2][W][MT][8] slice sums, by parity */

  if(wave == W){
    /* ---------------------------------------------------------------- control wave */
    int par = 0;
    for(int s = 0; s < nS; ++s){
      if(s > 0) kt_plan_barrier(ctr, (unsigned)(s - 1), (unsigned)G, lane);
      __syncthreads();                                           /* B1: stage s may start */
      const KtPStage& S = kt_stage_at(plan, s);
      for(int i = b; i < S.nitems; i += G){
        {
          const int t0 = 0, nt = S.M;
          __syncthreads();                                       /* B2: the slice sums of item i are in LDS */
          for(int p = lane; p < S.rgpi * 8; p += 64){
            const int ri = p >> 3, rr = p & 7, rg = i * S.rgpi + ri;
            if(rg < S.ngroups){
              int mi = 0;
              if(S.nmat > 1 && rg >= S.mat[1].rg0) mi = 1;
              if(S.nmat > 2 && rg >= S.mat[2].rg0) mi = 2;
              const KtMat& m = S.mat[mi];
              const int row = (rg - m.rg0) * KT_RG + rr;
              if(row < m.R){
                for(int t = 0; t < nt; ++t){
                  const float* q = red + ((size_t)(par * W + ri * S.KS) * MT + t) * 8 + rr;
                  float v = q[0];
                  for(int k = 1; k < S.KS; ++k) v += q[(size_t)k * MT * 8];
                  kt_stg<float>(m.y + (long long)(t0 + t) * m.ldy + row, v);
                }
              }
            }
          }
          par ^= 1;
        }
      }
    }
    return;
  }

  /* ------------------------------------------------------------------ data wave dw */
  const int dw = wave;
  uint8_t* xw = kt_lds + (size_t)dw * F::XW;
  int par = 0, s_done = -1;                                       /* stages whose B1 this wave has passed */
  KtStep WA[SL], WB[SL];

  /* the weight loads of a task (every offset first, then every load; a lane without a unit reads offset 0) */
  auto load_w = [&](const KtTask& t, KtStep (&w)[SL]) __attribute__((always_inline)) {
    const KtPStage& S = kt_stage_at(plan, t.s);
    const int ri = dw / S.KS, ks = dw - ri * S.KS, rg = t.i * S.rgpi + ri;
    const bool act = ri < S.rgpi && rg < S.ngroups;
    int mi = 0;
    if(act && S.nmat > 1 && rg >= S.mat[1].rg0) mi = 1;
    if(act && S.nmat > 2 && rg >= S.mat[2].rg0) mi = 2;
    const KtMat& m = S.mat[mi];
    const int NU = S.NU, St = kt_steps(NU), s_lo = ks * St / S.KS, ns = (ks + 1) * St / S.KS - s_lo;
    const int lrg = rg - m.rg0;
    unsigned o0[SL], o1[SL], os[SL];
#pragma unroll
    for(int j = 0; j < SL; ++j){
      const int st = s_lo + j, u = st * KT_KL + c;
      const bool ok = act && j < ns && u < NU;
      o0[j] = ok ? (unsigned)kt_widx(NU, lrg, st, 0, c, r) : 0u;
      o1[j] = ok ? (unsigned)kt_widx(NU, lrg, st, 1, c, r) : 0u;
      os[j] = ok ? (unsigned)kt_sidx(NU, lrg, u, r) : 0u;
    }
    const uint4* wb = (const uint4*)m.codes;
    const uint16_t* sb = m.scales;
#pragma unroll
    for(int j = 0; j < SL; ++j){
      w[j].c0 = kt_ldnt_g(wb + o0[j]);
      w[j].c1 = kt_ldnt_g(wb + o1[j]);
      w[j].hs = kt_ldg<uint16_t>(sb + os[j]);
    }
  };

  /* run task t with weights w; the next task's weights go to wn */
  auto run = [&](const KtTask& t, const KtStep (&w)[SL], const KtTask& tn, KtStep (&wn)[SL]) __attribute__((always_inline)) {
    while(s_done < t.s){ __syncthreads(); ++s_done; }             /* B1 of every stage up to t's */
    const KtPStage& S = kt_stage_at(plan, t.s);
    const int ri = dw / S.KS, ks = dw - ri * S.KS, rg = t.i * S.rgpi + ri;
    const bool act = ri < S.rgpi && rg < S.ngroups;              /* wave-uniform */
    const int NU = S.NU, St = kt_steps(NU), s_lo = ks * St / S.KS, ns = (ks + 1) * St / S.KS - s_lo;
    {                                                               /* one pass: M <= MT tokens */
      const int t0 = 0, nt = S.M;
      uint32_t sa[2][SL][MT];
      uint4 stg[SL][MT];
      const int o = lane * 16;
#pragma unroll
      for(int j = 0; j < SL; ++j){
        const int st = s_lo + (j < ns ? j : 0), u = st * KT_KL + c, uu = (j < ns && u < NU) ? u : 0;
        const int nc = NU - st * KT_KL < KT_KL ? NU - st * KT_KL : KT_KL;
#pragma unroll
        for(int tt = 0; tt < MT; ++tt){
          const int n = t0 + (tt < nt ? tt : 0);
          sa[0][j][tt] = kt_ldg<uint32_t>(S.xs + (long long)n * S.ldxs + uu);
          sa[1][j][tt] = kt_ldg<uint32_t>(S.xa + (long long)n * S.ldxs + uu);
          const int oc = o < nc * UW ? o : 0;
          stg[j][tt] = kt_ldg4(S.xq + (long long)n * S.ldq + (long long)st * KT_KL * UW + oc);
        }
      }
      kt_pin<SL * MT>(&stg[0][0], &sa[0][0][0]);
      const int lo = (o / UW) * UP + o % UW;
#pragma unroll
      for(int j = 0; j < SL; ++j)
#pragma unroll
        for(int tt = 0; tt < MT; ++tt)
          *(uint4*)(xw + (j * MT + tt) * KT_KL * UP + lo) = stg[j][tt];
      /* the next task's weights: issued after this task's activations have arrived (a wait for those is then a wait
         for nothing else) and before its compute, so they travel during this task and the barriers that follow */
      if(tn.s < nS) load_w(tn, wn);
      kt_wave_sync();
      if(act){
        float acc[MT];
#pragma unroll
        for(int tt = 0; tt < MT; ++tt) acc[tt] = 0.0f;
#pragma unroll
        for(int j = 0; j < SL; ++j){
          const int u = (s_lo + j) * KT_KL + c;
          if(j < ns){                                               /* wave-uniform */
            const bool uok = u < NU;
            const float d = uok ? kt_h2f(w[j].hs) : 0.0f;
#pragma unroll
            for(int tt = 0; tt < MT; ++tt){
              if(tt < nt){
                int v = kt_unit_lds<KT_FMT_TERN>(w[j].c0, w[j].c1, xw + ((j * MT + tt) * KT_KL + (uok ? c : 0)) * UP)
                        - (int)sa[1][j][tt];
                v = uok ? v : 0;
                acc[tt] = fmaf((float)v, __uint_as_float(sa[0][j][tt]) * d, acc[tt]);
              }
            }
          }
        }
#pragma unroll
        for(int tt = 0; tt < MT; ++tt){
          const float y = kt_row_sum(acc[tt]);
          if(c == 0) red[((size_t)(par * W + dw) * MT + tt) * 8 + r] = y;
        }
      }
      kt_wave_sync();                                               /* the staging is rewritten next */
      __syncthreads();                                              /* B2 */
      par ^= 1;
    }
  };

  KtTask t = kt_first_task(plan, nS, b);
  if(t.s < nS) load_w(t, WA);
  while(t.s < nS){
    const KtTask u = kt_next_task(plan, nS, b, G, t);
    run(t, WA, u, WB);
    if(u.s >= nS) break;
    const KtTask v = kt_next_task(plan, nS, b, G, u);
    run(u, WB, v, WA);
    t = v;
  }
  while(s_done < nS - 1){ __syncthreads(); ++s_done; }              /* the remaining stages' B1 */
}

extern "C" __global__ void k_plan_reset(unsigned* ctr, int n){
  for(int i = threadIdx.x; i < n; i += blockDim.x) ctr[i] = 0u;
}

template __global__ void k_plan<1>(const uint8_t*, unsigned*);
template __global__ void k_plan<2>(const uint8_t*, unsigned*);
template __global__ void k_plan<4>(const uint8_t*, unsigned*);
