/* kt_plan.h - what the decode-plan executors (kt_plan.hip, kt_splan.hip) share: the stage table and the grid
   barrier */
#pragma once
#include "kt_gemv.h"

#ifndef KT_SPIN_MAX
#define KT_SPIN_MAX (1u << 18)        /* spin iterations of one barrier (each at least one memory round trip) */
#endif

__device__ __forceinline__ const KtPStage& kt_stage_at(const uint8_t* plan, int s){
  return ((const KtPStage*)(plan + KT_PLAN_HDR))[s];
}

/* the grid barrier of the control wave before stage k + 1 (k = 0, 1, ...). Block b arrives on counter b % 32 (32
   counters on their own 128-byte lines, so arrivals do not queue on one address); lanes 0..31 then poll one counter
   each until every counter has reached its count for barrier k ((k + 1) x its blocks: counts only grow, and no
   block arrives at barrier k + 1 before all have arrived at k). No cache-wide maintenance: what crosses stages is
   made coherent where it is written and read instead (agent-scope stores of the output rows; agent-scope loads of
   a stage's inputs when they overlap an earlier stage's outputs). The fences here are workgroup scope and do not
   wait for the wave's outstanding stores: a caller whose stores must be visible to the other blocks waits for them
   (s_waitcnt vmcnt(0)) before it arrives. */
__device__ __forceinline__ void kt_plan_barrier(unsigned* ctr, unsigned k, unsigned G, int lane){
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
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
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

/* the block barrier of the plan: LDS traffic of the wave done, then s_barrier. Unlike __syncthreads it does not
   wait for the wave's global loads and stores (the data waves' prefetch, the control wave's output stores), which
   nothing across this barrier needs: the slice sums meet in LDS, and the stage ordering is the grid barrier's. */
__device__ __forceinline__ void kt_block_sync(){
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

