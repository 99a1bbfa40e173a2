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
   The control wave issues no weight loads, so its waits are for nothing but its own stores and atomics. The plan (header, stages) is read-only in the launch and the barrier counters and status word come as a
   separate argument, so the stage fields are scalar loads. A spin that runs out of iterations sets the plan's status word and every later barrier then passes at
   once, so a failed plan ends instead of hanging (kt_plan_status reports it). */
#include "kt_gemv.h"

#include "kt_plan.h"

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
      /* the block's rows of stage s - 1 are complete in memory before it arrives: the agent-scope stores are
         relaxed and a workgroup-scope fence does not wait for them (the control wave issues no other memory
         operations, so this waits for nothing else) */
      if(s > 0){ __builtin_amdgcn_s_waitcnt(0); kt_plan_barrier(ctr, (unsigned)(s - 1), (unsigned)G, lane); }
      kt_block_sync();                                           /* B1: stage s may start */
      const KtPStage& S = kt_stage_at(plan, s);
      for(int i = b; i < S.nitems; i += G){
        {
          const int t0 = 0, nt = S.M;
          kt_block_sync();                                       /* B2: the slice sums of item i are in LDS */
          const int t = lane >> 3, rr = lane & 7;                /* lane = 8 t + r: token t, row r of a group */
          for(int ri = 0; ri < S.rgpi; ++ri){                    /* uniform: the matrix fields are scalar */
            const int rg = i * S.rgpi + ri;
            if(rg >= S.ngroups) break;
            int mi = 0;
            if(S.nmat > 1 && rg >= S.mat[1].rg0) mi = 1;
            if(S.nmat > 2 && rg >= S.mat[2].rg0) mi = 2;
            const KtMat& m = S.mat[__builtin_amdgcn_readfirstlane(mi)];
            const int row = (rg - m.rg0) * KT_RG + rr;
            if(t < nt && row < m.R){
              const float* q = red + ((size_t)(par * W + ri * S.KS) * MT + t) * 8 + rr;
              float v = q[0];
              for(int k = 1; k < S.KS; ++k) v += q[(size_t)k * MT * 8];
              __hip_atomic_store((KT_G float*)(m.y + (long long)(t0 + t) * m.ldy + row), v, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
            }
          }
          par ^= 1;
        }
      }
    }
    return;
  }

  /* ------------------------------------------------------------------ data wave dw
     A wave's K slice (dw % KS) is the same for every item of a stage, so its activations are staged once per stage
     (into the wave's LDS region, the unit scales and sums into registers). Weights run through a ring of three
     register sets: while task k computes, tasks k + 1 and k + 2 are in flight, and the set of task k is refilled
     with task k + 3 after it. The activations of the next stage are fetched with the weights that first reach it,
     unless that stage reads what an earlier stage writes (then after its barrier). */
  const int dw = wave;
  uint8_t* xw = kt_lds + (size_t)dw * F::XW;
  int par = 0, s_done = -1, s_in = -1, s_pend = -1;             /* B1 passed; stage staged; stage fetched early */
  KtStep W0[SL], W1[SL], W2[SL];
  uint32_t saC[2][SL][MT], saP[2][SL][MT];                      /* unit scale (f32 bits) and sum: staged, early */
  uint4 stgP[SL][MT];

  /* the loads of stage s's activations for this wave's slice: its steps' rows (16 bytes a lane) and unit values */
  auto load_x = [&](int s, uint4 (&stg)[SL][MT], uint32_t (&sa)[2][SL][MT]) __attribute__((always_inline)) {
    const KtPStage& S = kt_stage_at(plan, s);
    const int ks = dw % S.KS, NU = S.NU, St = kt_steps(NU), s_lo = ks * St / S.KS, ns = (ks + 1) * St / S.KS - s_lo;
    const int o = lane * 16;
#pragma unroll
    for(int j = 0; j < SL; ++j){
      const int st = s_lo + (j < ns ? j : 0), u = st * KT_KL + c, uu = (j < ns && u < NU) ? u : 0;
      const int nc = NU - st * KT_KL < KT_KL ? NU - st * KT_KL : KT_KL;
#pragma unroll
      for(int tt = 0; tt < MT; ++tt){
        const int n = tt < S.M ? tt : 0;
        const int oc = o < nc * UW ? o : 0;
        const float* px = S.xs + (long long)n * S.ldxs + uu;
        const int* pa = S.xa + (long long)n * S.ldxs + uu;
        const int8_t* pq = S.xq + (long long)n * S.ldq + (long long)st * KT_KL * UW + oc;
        if(S.coh){                                                  /* written in this launch: coherent loads */
          sa[0][j][tt] = __hip_atomic_load((const KT_G unsigned*)px, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          sa[1][j][tt] = __hip_atomic_load((const KT_G unsigned*)pa, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          const KT_G unsigned* q4 = (const KT_G unsigned*)pq;
          stg[j][tt] = make_uint4(__hip_atomic_load(q4, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                                  __hip_atomic_load(q4 + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                                  __hip_atomic_load(q4 + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                                  __hip_atomic_load(q4 + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        } else {
          sa[0][j][tt] = kt_ldg<uint32_t>(px);
          sa[1][j][tt] = kt_ldg<uint32_t>(pa);
          stg[j][tt] = kt_ldg4(pq);
        }
      }
    }
  };
  /* the staged rows into the wave's LDS region (every slot written; the ones of absent units are never read) */
  auto put_x = [&](const uint4 (&stg)[SL][MT]) __attribute__((always_inline)) {
    const int o = lane * 16, lo = (o / UW) * UP + o % UW;
#pragma unroll
    for(int j = 0; j < SL; ++j)
#pragma unroll
      for(int tt = 0; tt < MT; ++tt)
        *(uint4*)(xw + (j * MT + tt) * KT_KL * UP + lo) = stg[j][tt];
    kt_wave_sync();
  };

  /* the weight loads of a task (every offset first, then every load; a lane without a unit reads offset 0) */
  auto load_w = [&](const KtTask& t, KtStep (&w)[SL]) __attribute__((always_inline)) {
    const bool live = t.s < nS;                                     /* past the last task: the same loads, offset 0 */
    const KtPStage& S = kt_stage_at(plan, live ? t.s : 0);
    const int ri = dw / S.KS, ks = dw - ri * S.KS, rg = t.i * S.rgpi + ri;
    const bool act = live && ri < S.rgpi && rg < S.ngroups;
    int mi = 0;
    if(act && S.nmat > 1 && rg >= S.mat[1].rg0) mi = 1;
    if(act && S.nmat > 2 && rg >= S.mat[2].rg0) mi = 2;
    const KtMat& m = S.mat[__builtin_amdgcn_readfirstlane(mi)];
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
  /* a task's weights (the same loads when there is no task: every path issues as many, so the compiler's wait
     counts for the ring stay exact), and the activations of its stage when it is a later stage seen ahead */
  auto prefetch = [&](const KtTask& t, KtStep (&w)[SL]) __attribute__((always_inline)) {
    load_w(t, w);                                                   /* always issued: exact wait counts */
    if(t.s < nS && t.s != s_in && s_pend < 0 && !kt_stage_at(plan, t.s).coh){
      load_x(t.s, stgP, saP);
      s_pend = t.s;
    }
  };

  /* run task t with weights w; then refill w with task tr */
  auto run = [&](const KtTask& t, KtStep (&w)[SL], const KtTask& tr) __attribute__((always_inline)) {
    const KtPStage& S = kt_stage_at(plan, t.s);
    if(t.s != s_in){                                                /* the first task of a stage for this wave */
      while(s_done < t.s){ kt_block_sync(); ++s_done; }           /* B1 of every stage up to t's */
      if(s_pend == t.s){
        put_x(stgP);
#pragma unroll
        for(int j = 0; j < SL; ++j)
#pragma unroll
          for(int tt = 0; tt < MT; ++tt){ saC[0][j][tt] = saP[0][j][tt]; saC[1][j][tt] = saP[1][j][tt]; }
        s_pend = -1;
      } else {
        uint4 stg[SL][MT];
        load_x(t.s, stg, saC);
        put_x(stg);
      }
      s_in = t.s;
    }
    const int ri = dw / S.KS, ks = dw - ri * S.KS, rg = t.i * S.rgpi + ri;
    const bool act = ri < S.rgpi && rg < S.ngroups;                /* wave-uniform */
    const int NU = S.NU, St = kt_steps(NU), s_lo = ks * St / S.KS, ns = (ks + 1) * St / S.KS - s_lo;
    const int nt = S.M;
    if(act){
      float acc[MT];
#pragma unroll
      for(int tt = 0; tt < MT; ++tt) acc[tt] = 0.0f;
#pragma unroll
      for(int j = 0; j < SL; ++j){
        const int u = (s_lo + j) * KT_KL + c;
        if(j < ns){                                                 /* wave-uniform */
          const bool uok = u < NU;
          const float d = uok ? kt_h2f(w[j].hs) : 0.0f;
#pragma unroll
          for(int tt = 0; tt < MT; ++tt){
            if(tt < nt){
              int v = kt_unit_lds<KT_FMT_TERN>(w[j].c0, w[j].c1, xw + ((j * MT + tt) * KT_KL + (uok ? c : 0)) * UP)
                      - (int)saC[1][j][tt];
              v = uok ? v : 0;
              acc[tt] = fmaf((float)v, __uint_as_float(saC[0][j][tt]) * d, acc[tt]);
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
    kt_block_sync();                                                /* B2 */
    par ^= 1;
    prefetch(tr, w);
  };

  KtTask t0 = kt_first_task(plan, nS, b);
  KtTask t1 = kt_next_task(plan, nS, b, G, t0);
  KtTask t2 = kt_next_task(plan, nS, b, G, t1);
  prefetch(t0, W0);
  prefetch(t1, W1);
  prefetch(t2, W2);
  while(t0.s < nS){
    const KtTask t3 = kt_next_task(plan, nS, b, G, t2);
    run(t0, W0, t3);
    if(t1.s >= nS) break;
    const KtTask t4 = kt_next_task(plan, nS, b, G, t3);
    run(t1, W1, t4);
    if(t2.s >= nS) break;
    const KtTask t5 = kt_next_task(plan, nS, b, G, t4);
    run(t2, W2, t5);
    t0 = t3; t1 = t4; t2 = t5;
  }
  while(s_done < nS - 1){ kt_block_sync(); ++s_done; }              /* the remaining stages' B1 */
}

/* the barrier's used words (word 0 of each of its n lines) to zero before a run */
extern "C" __global__ void k_plan_reset(unsigned* ctr, int n){
  for(int i = threadIdx.x; i < n; i += blockDim.x) ctr[i * KT_BAR_LINE] = 0u;
}

template __global__ void k_plan<1>(const uint8_t*, unsigned*);
template __global__ void k_plan<2>(const uint8_t*, unsigned*);
template __global__ void k_plan<4>(const uint8_t*, unsigned*);
