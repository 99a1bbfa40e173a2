/* kt_plan.hip - the decode plan executor: a sequence of ternary products (the per-layer launches of a decode step,
   spec.py:619-673: q/k/v, o, gate/up, down, ...) run by one persistent launch, one block per CU.

   Work (assigned by kt_plan_build). Stage s has N_s row groups (8 rows of all its matrices) and KS_s K slices (the
   decode product's slices, kt_kslices). Block b takes the row groups p, p + G, p + 2 G, ... with p = (b - off_s)
   mod G; off_s advances by N_s mod G from stage to stage, so the blocks that take one row group more rotate. The
   block's tasks of a stage are its (row group, slice) pairs, dealt to its data waves in turn, the deal carried on
   from stage to stage. A data wave's work is a list of step records (one 16-byte record per 8-row x 8-unit step:
   the step's code address, its scale offset, its step index and unit count, slice start and end, the slot of the
   slice sum, the stage), in stage order.

   A data wave reads its records KT_RING at a time (one window per pass of its loop, two passes ahead) and walks
   them through a ring of KT_RING register sets of weights: while it computes
   step k, the loads of steps k + 1 .. k + KT_RING - 1 are in flight, across stage ends (weights never depend on
   earlier stages), so the weight stream keeps going through the stage barriers. Each step is computed exactly as
   k_gemv_flat computes it: lane 8 c + r takes unit 8 step + c of row r, chains its units of the slice with fmaf in
   order, and the 8 lanes of a row meet in the xor butterfly at the slice's end; the slice sum goes to LDS.

   The control wave (wave KT_PW) stages each stage's activations (int8 rows, XS and XA per unit) in LDS, adds the KS
   slice sums of each row in slice order once the data waves are done with the stage, stores the row (agent-scope
   stores, so other XCDs read it from memory), waits for its stores and arrives at the grid barrier; after the
   barrier it releases the block into the next stage. With two activation buffers the next stage's activations are
   staged while the current one computes, unless they overlap an earlier stage's outputs (then they are read with
   coherent loads after the barrier). Every output bit equals the single-launch product's (same units, lanes,
   chains, butterfly and slice order), and a stage sees everything earlier stages wrote: the ordering and
   visibility of separate stream-ordered launches.

   Block synchronisation, by words in LDS: the control wave publishes the stage whose activations are staged (the
   data waves start a stage once it is published), and each data wave publishes how many stages it has finished
   (a wave without a task in a stage finishes it when it moves past it); the control wave reduces stage s once
   every data wave has finished s + 1 stages. Neither side waits for the other's global memory traffic.
   A barrier spin that runs out of iterations sets the plan's status word and every later barrier then passes at
   once, so a failed plan ends instead of hanging (kt_plan_status reports it). */
#include "kt_gemv.h"

#ifndef KT_SPIN_MAX
#define KT_SPIN_MAX (1u << 18)        /* spin iterations of one barrier (each at least one memory round trip) */
#endif
#ifndef KT_RING
#define KT_RING 8                     /* steps of weights in flight a data wave */
#endif
#define KT_PW KT_PLAN_WAVES
/* measurement builds only: KT_PLAN_TRACE records s_memrealtime at the stage events of every block after the barrier
   words ([G][nS][16] words: control wave 0..4, data wave w 8 + w) */
#ifdef KT_PLAN_TRACE
#define KT_TR(s, k) do { if(lane == 0) trace[((size_t)b * nS + (s)) * 16 + (k)] = (unsigned)__builtin_amdgcn_s_memrealtime(); } while(0)
#else
#define KT_TR(s, k) do { } while(0)
#endif
#ifndef KT_PLAN_ABL
#define KT_PLAN_ABL 0                 /* measurement builds only: 1 no products, 2 no grid barrier, 4 no row stores */
#endif

__device__ __forceinline__ const KtPStage& kt_stage_at(const uint8_t* plan, int s){
  return ((const KtPStage*)(plan + KT_PLAN_HDR))[s];
}

/* the grid barrier of the control wave after stage k (k = 0, 1, ...). Block b arrives on counter b % 32 (32
   counters on their own 128-byte lines, so arrivals do not queue on one address); lanes 0..31 then poll one counter
   each until every counter has reached its count for barrier k ((k + 1) x its blocks: counts only grow, and no
   block arrives at barrier k + 1 before all have arrived at k). No cache-wide maintenance: what crosses stages is
   made coherent where it is written and read (agent-scope stores of the rows; agent-scope loads of a stage's
   inputs when they overlap an earlier stage's outputs); the wave waits for its own stores before it arrives. */
__device__ __forceinline__ void kt_plan_barrier(unsigned* ctr, unsigned k, unsigned G, int lane){
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  unsigned* status = ctr + KT_BAR_STATUS * 32;
  if(lane == 0)
    __hip_atomic_fetch_add(ctr + (KT_BAR_SUB + blockIdx.x % KT_BAR_SHARDS) * 32, 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  if(__hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u){
    const unsigned want = lane < KT_BAR_SHARDS ? (k + 1u) * ((G - lane + KT_BAR_SHARDS - 1) / KT_BAR_SHARDS) : 0u;
    unsigned* mine = ctr + (KT_BAR_SUB + (lane < KT_BAR_SHARDS ? lane : 0)) * 32;
    for(unsigned n = 0;; ++n){
      const unsigned v = lane < KT_BAR_SHARDS ? __hip_atomic_load(mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
      if(__ballot(v < want) == 0) break;
      if(n == KT_SPIN_MAX){
        if(lane == 0) __hip_atomic_fetch_or(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
}

/* the first block barrier (the LDS tables and flags are set): the wave's LDS traffic done, then s_barrier */
__device__ __forceinline__ void kt_block_sync(){
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

/* block-level signals in LDS (KT_FLAGS bytes): word 0 is the last stage whose activations the control wave has
   staged (a release store after its LDS writes); word 8 + w is the number of stages data wave w has finished (a
   release store after its slice sums are written). The waits are acquire loads, so no read of the staged data or
   of the sums moves above them. */
#define KT_FLAGS 64
__device__ __forceinline__ void kt_publish(int* flag, int s, int lane){
  if(lane == 0) __hip_atomic_store(&flag[0], s, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void kt_wait_ready(int* flag, int s){
  while(__hip_atomic_load(&flag[0], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < s) __builtin_amdgcn_s_sleep(1);
}
__device__ __forceinline__ void kt_signal(int* flag, int w, int n, int lane){
  if(lane == 0) __hip_atomic_store(&flag[8 + w], n, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
/* the control wave: until every data wave has finished n stages (lane w < KT_PW reads wave w's word) */
__device__ __forceinline__ void kt_wait_done(int* flag, int n, int lane){
  for(;;){
    const int v = lane < KT_PW ? __hip_atomic_load(&flag[8 + lane], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) : n;
    if(__ballot(v < n) == 0) break;
    __builtin_amdgcn_s_sleep(1);
  }
}

__device__ __forceinline__ int kt_u(int v){ return __builtin_amdgcn_readfirstlane(v); }

/* the fixed xor butterfly over the 8 k-lanes of a row (lane bits 3..5), with the same additions as kt_row_sum:
   xor 8 inside a row of 16 lanes (DPP rotate by 8); xor 16 and xor 32 by the gfx950 lane swaps. A swap of v with
   itself returns (v with odd rows / upper half replaced by the even rows / lower half, v with even rows / lower
   half replaced by the odd rows / upper half): the partner of a lane is the second result in the lower row / half
   and the first in the upper one. */
__device__ __forceinline__ float kt_row_sum_x(float v, int lane){
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false));  /* row_ror:8 */
  {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
    v += __int_as_float((int)((lane & 16) ? p[0] : p[1]));
  }
  {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
    v += __int_as_float((int)((lane & 32) ? p[0] : p[1]));
  }
  return v;
}

template <int MT>
__global__ void __launch_bounds__(64 * (KT_PW + 1)) k_plan(const uint8_t* __restrict__ plan, unsigned* __restrict__ ctr){
  extern __shared__ __attribute__((aligned(16))) uint8_t kt_lds[];
  constexpr int UW = 128, UP = UW + 16;
  const KtPlanHdr& H = *(const KtPlanHdr*)plan;
  const int nS = H.nstages, G = H.G, NB = H.NB, NUX = H.NUX, M = H.M, b = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int r = lane & 7, c = lane >> 3;
  /* LDS: the flags (KT_FLAGS bytes), the stages' row tables [nS], activations [NB][MT][NUX][UP], unit scale and sum
     [NB][MT][NUX][2], slice sums [RED][MT][8] */
  int* flag = (int*)kt_lds;
#ifdef KT_PLAN_TRACE
  unsigned* trace = ctr + KT_BAR_WORDS;
#endif
  KtPCtl* T = (KtPCtl*)(kt_lds + KT_FLAGS);
  uint8_t* xb = kt_lds + KT_FLAGS + (size_t)nS * sizeof(KtPCtl);
  int* xsa = (int*)(xb + (size_t)NB * MT * NUX * UP);
  float* red = (float*)(xsa + (size_t)NB * MT * NUX * 2);
  {
    /* the row tables into LDS, by every wave */
    const uint4* src = (const uint4*)(plan + kt_plan_ctl_off(nS));
    for(int i = threadIdx.x; i < nS * (int)(sizeof(KtPCtl) / 16); i += 64 * (KT_PW + 1))
      ((uint4*)T)[i] = kt_ldg4(src + i);
  }

  if(wave == KT_PW){
    /* ---------------------------------------------------------------- control wave */
    /* stage s's activations into buffer buf: 16 bytes a lane a load, 8 loads in flight, then their LDS writes */
    auto stage_x = [&](int s, int buf) __attribute__((always_inline)) {
      const KtPStage& S = kt_stage_at(plan, s);
      const int NU = S.NU, n16 = NU * 8;
      const bool coh = S.coh != 0;
      for(int t = 0; t < M; ++t){
        const int8_t* src = S.xq + (long long)t * S.ldq;
        uint8_t* dst = xb + (size_t)(buf * MT + t) * NUX * UP;
        for(int i0 = 0; i0 < n16; i0 += 64 * 8){
          uint4 v[8];
#pragma unroll
          for(int k = 0; k < 8; ++k){
            const int i = i0 + k * 64 + lane, ii = i < n16 ? i : 0;
            const KT_G unsigned* q4 = (const KT_G unsigned*)(src + ii * 16);
            if(coh)
              v[k] = make_uint4(__hip_atomic_load(q4, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                                __hip_atomic_load(q4 + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                                __hip_atomic_load(q4 + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                                __hip_atomic_load(q4 + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            else
              v[k] = kt_ldg4(src + ii * 16);
          }
#pragma unroll
          for(int k = 0; k < 8; ++k){
            const int i = i0 + k * 64 + lane;
            if(i < n16) *(uint4*)(dst + (i >> 3) * UP + (i & 7) * 16) = v[k];
          }
        }
        int* da = xsa + (size_t)(buf * MT + t) * NUX * 2;
        for(int u = lane; u < NU; u += 64){
          const long long o = (long long)t * S.ldxs + u;
          unsigned xs, xa;
          if(coh){
            xs = __hip_atomic_load((const KT_G unsigned*)(S.xs + o), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            xa = __hip_atomic_load((const KT_G unsigned*)(S.xa + o), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          } else {
            xs = kt_ldg<unsigned>(S.xs + o);
            xa = kt_ldg<unsigned>(S.xa + o);
          }
          da[2 * u] = (int)xs;
          da[2 * u + 1] = (int)xa;
        }
      }
    };
    if(lane < 16) flag[lane] = lane == 0 ? -1 : 0;                  /* before the first block barrier */
    kt_block_sync();                                                /* the flags and tables are set */
    stage_x(0, 0);
    kt_publish(flag, 0, lane);
    for(int s = 0; s < nS; ++s){
      const KtPCtl& C = T[s];
      const bool more = s + 1 < nS;
      const bool early = more && NB == 2 && !kt_u(T[s + 1].coh);
      if(early) stage_x(s + 1, (s + 1) & 1);                        /* while the data waves compute stage s */
      KT_TR(s, 0);
      kt_wait_done(flag, s + 1, lane);                              /* every data wave is done with stage s */
      KT_TR(s, 1);
      /* the block's rows of stage s: lane = 8 (row group slot) + row, 8 row groups a pass */
      const int off = kt_u(C.off), KS = kt_u(C.KS), N = kt_u(C.ngroups), rg1 = kt_u(C.rg1), rg2 = kt_u(C.rg2);
      int p = b - off;
      if(p < 0) p += G;
      const int cnt = p < N ? (N - 1 - p) / G + 1 : 0;
      for(int k0 = 0; k0 < cnt; k0 += 8){
        const int rgk = k0 + (lane >> 3), rr = lane & 7;
        if(rgk < cnt){
          const int rg = p + rgk * G;
          const int mi = rg >= rg2 ? 2 : rg >= rg1 ? 1 : 0;
          float* y = (float*)(mi == 2 ? C.y[2] : mi == 1 ? C.y[1] : C.y[0]);
          const int R = mi == 2 ? C.R[2] : mi == 1 ? C.R[1] : C.R[0];
          const int row = (rg - (mi == 2 ? rg2 : mi == 1 ? rg1 : 0)) * KT_RG + rr;
          if(row < R && !(KT_PLAN_ABL & 4)){
            for(int t = 0; t < M; ++t){
              const float* q = red + ((size_t)rgk * KS * MT + t) * 8 + rr;
              float v = q[0];
              for(int k = 1; k < KS; ++k) v += q[(size_t)k * MT * 8];
              __hip_atomic_store((KT_G float*)(y + (long long)t * R + row), v, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
            }
          }
        }
      }
      KT_TR(s, 2);
      if(more){
        if(!(KT_PLAN_ABL & 2)) kt_plan_barrier(ctr, (unsigned)s, (unsigned)G, lane);
        KT_TR(s, 3);
        if(!early) stage_x(s + 1, NB == 2 ? (s + 1) & 1 : 0);
        kt_publish(flag, s + 1, lane);
        KT_TR(s, 4);
      }
    }
    return;
  }

  /* ------------------------------------------------------------------ data wave w */
  const int w = wave;
  const unsigned* idx = (const unsigned*)(plan + kt_plan_idx_off(nS));
  const uint4* rec = (const uint4*)(plan + kt_plan_rec_off(nS)) + kt_ldg<unsigned>(idx + b * KT_PW + w);
  const unsigned lo0 = (unsigned)(c * 8 + r) * 16u, lso = (unsigned)(c * 8 + r) * 2u;   /* the lane's offsets */
  /* record j of a window of KT_RING (lane j holds it; the other lanes hold copies) */
  struct KtR { uint64_t codes; int soff; unsigned bits; };
  /* one step's weights as loaded (raw registers: nothing reads them before the step's wait) */
  struct KtRaw { kt_u32x4 c0, c1; unsigned hs; };
  /* the loads of step record q (a lane without a unit reads the step's first 16 bytes). They are issued by asm, so
     the compiler places no waits for them: each step waits explicitly, with the exact count of the loop's fixed
     load pattern, and takes the step's registers as operands of the wait, so no use moves above it. */
  auto load = [&](const KtR& q, KtRaw& st) __attribute__((always_inline)) {
    const int nc = ((q.bits >> 5) & 7) + 1;
    const bool ok = c < nc;
    const uint8_t* base = (const uint8_t*)q.codes;
    const unsigned o0 = ok ? lo0 : 0u, o1 = ok ? lo0 + (unsigned)nc * 128u : 0u, os = ok ? lso : 0u;
    asm volatile("global_load_dwordx4 %0, %1, off nt" : "=v"(st.c0) : "v"(base + o0));
    asm volatile("global_load_dwordx4 %0, %1, off nt" : "=v"(st.c1) : "v"(base + o1));
    asm volatile("global_load_ushort %0, %1, off" : "=v"(st.hs) : "v"(base + (long long)q.soff + os));
  };
  auto ldrec = [&](const uint4* p) __attribute__((always_inline)) -> kt_u32x4 {
    kt_u32x4 v;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p));
    return v;
  };
  auto get = [&](const kt_u32x4& R, int j) __attribute__((always_inline)) -> KtR {
    KtR q;
    /* readlane returns int: each half goes through unsigned, so the low half is not sign-extended */
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)R.x, j), hi = (unsigned)__builtin_amdgcn_readlane((int)R.y, j);
    q.codes = (uint64_t)lo | (uint64_t)hi << 32;
    q.soff = __builtin_amdgcn_readlane((int)R.z, j);
    q.bits = (unsigned)__builtin_amdgcn_readlane((int)R.w, j);
    return q;
  };

  KtRaw ring[KT_RING];
  unsigned rbits[KT_RING];                                         /* the record bits of the ring's steps */
  kt_block_sync();                                                 /* the flags and tables are set */
  const int rl = lane & (KT_RING - 1);
  /* the first two record windows, both complete before the ring is filled: the loop's first pass refills from
     window 1 and its waits count only the ring's loads and the window loaded at the pass's start */
  kt_u32x4 RB = ldrec(rec + KT_RING + rl), RA;
  {
    kt_u32x4 R0 = ldrec(rec + rl);
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(R0), "+v"(RB));
#pragma unroll
    for(int j = 0; j < KT_RING; ++j){
      const KtR q = get(R0, j);
      load(q, ring[j]);
      rbits[j] = q.bits;
    }
  }
  /* The loop's load pattern is fixed: a pass issues one record window, then per step three weight loads. Before
     step j of a pass, the loads issued after the step's own (made in the previous pass) are the 3 (KT_RING - 1 - j)
     of that pass's later steps, the window and the 3 j of this pass: 3 KT_RING - 2 in all, whatever j. Passes go in
     pairs over two window registers: pass i refills from window i + 1 (loaded at the start of pass i - 1, so done
     by then as well; window 1 before the loop) and loads window i + 2 into the register of window i. A pass that
     meets the end has loaded records up to 3 windows past its own: the lists are padded for that. */
  int rdy = -1;                                                    /* highest stage seen staged */
  float acc[MT];
#pragma unroll
  for(int t = 0; t < MT; ++t) acc[t] = 0.0f;
  auto pass = [&](kt_u32x4& Rc) __attribute__((always_inline)) -> bool {
#pragma unroll
    for(int j = 0; j < KT_RING; ++j){
      KtRaw& wj = ring[j];
      static_assert(3 * KT_RING - 2 <= 63, "vmcnt range");
      if(j == 0)
        asm volatile("s_waitcnt vmcnt(%3)" : "+v"(wj.c0), "+v"(wj.c1), "+v"(wj.hs) : "n"(3 * KT_RING - 2), "v"(Rc));
      else
        asm volatile("s_waitcnt vmcnt(%3)" : "+v"(wj.c0), "+v"(wj.c1), "+v"(wj.hs) : "n"(3 * KT_RING - 2));
      if(j == 0) asm volatile("" : "+v"(Rc));                      /* the window is read after the wait */
      const unsigned bits = rbits[j];
      const int st = (int)(bits >> 20);                            /* stage; nS: past the last record */
      if(st >= nS) return false;
      if(st > rdy){                                                /* the first step of a stage */
        kt_signal(flag, w, st, lane);                              /* earlier stages done (slice sums written) */
        kt_wait_ready(flag, st);                                   /* the stage's activations are staged */
        KT_TR(st, 8 + w);
        rdy = st;
      }
      const int nc = ((bits >> 5) & 7) + 1, sp = (int)(bits & 31), par = NB == 2 ? (st & 1) : 0;
      const bool uok = c < nc;
      const int uu = uok ? sp * KT_KL + c : 0;
      if(bits & 0x100u){
#pragma unroll
        for(int t = 0; t < MT; ++t) acc[t] = 0.0f;
      }
      const uint4 c0 = make_uint4(wj.c0.x, wj.c0.y, wj.c0.z, wj.c0.w), c1 = make_uint4(wj.c1.x, wj.c1.y, wj.c1.z, wj.c1.w);
      const float d = uok ? kt_h2f((uint16_t)wj.hs) : 0.0f;
#pragma unroll
      for(int t = 0; t < MT; ++t){
        if(KT_PLAN_ABL & 1){
          asm volatile("" :: "v"(c0.x), "v"(c1.x), "v"(d));
        } else if(t < M){
          const size_t xo = (size_t)(par * MT + t) * NUX + uu;
          const int2 sa = *(const int2*)(xsa + 2 * xo);
          int v = kt_unit_lds<KT_FMT_TERN>(c0, c1, xb + xo * UP) - sa.y;
          v = uok ? v : 0;
          acc[t] = fmaf((float)v, __int_as_float(sa.x) * d, acc[t]);
        }
      }
      if(bits & 0x200u){                                           /* the slice's last step */
        const int slot = (int)((bits >> 10) & 1023);
#pragma unroll
        for(int t = 0; t < MT; ++t){
          const float y = kt_row_sum_x(acc[t], lane);
          if(c == 0 && t < M) red[((size_t)slot * MT + t) * 8 + r] = y;
        }
      }
      const KtR q = get(Rc, j);                                    /* refill: the step KT_RING ahead */
      load(q, wj);
      rbits[j] = q.bits;
    }
    return true;
  };
  for(int k0 = 0;; k0 += 2 * KT_RING){
    RA = ldrec(rec + k0 + 2 * KT_RING + rl);
    if(!pass(RB)) break;
    RB = ldrec(rec + k0 + 3 * KT_RING + rl);
    if(!pass(RA)) break;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");                 /* nothing in flight at the end */
  kt_signal(flag, w, nS, lane);                                    /* every stage */
}

extern "C" __global__ void k_plan_reset(unsigned* ctr, int n){
  for(int i = threadIdx.x; i < n; i += blockDim.x) ctr[i] = 0u;
}

template __global__ void k_plan<1>(const uint8_t*, unsigned*);
template __global__ void k_plan<2>(const uint8_t*, unsigned*);
template __global__ void k_plan<4>(const uint8_t*, unsigned*);
