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

/* the grid barrier of the control wave before stage k + 1 (k = 0, 1, ...), a two-level tree over one-writer lines.
   Block b stores k + 1 to its own arrival line; the first block of each group of KT_BAR_FAN polls its group's lines
   (one lane each) and then stores k + 1 to the group line; every block polls the group lines (one lane each) until
   all hold at least k + 1 (values only grow, and no block arrives at barrier k + 1 before all have passed k). Two
   signal hops of about 0.6 us each; a flat barrier (every block polling every arrival) or one counter that all blocks
   add to queues at the memory side and takes 2.7-4 us on 256 blocks. No cache-wide maintenance: what crosses stages
   is made coherent where it is written and read instead (agent-scope stores of the output rows; agent-scope loads of
   a stage's inputs when they overlap an earlier stage's outputs). The fences here are workgroup scope and do not
   wait for the wave's outstanding stores: a caller whose stores must be visible to the other blocks waits for them
   (s_waitcnt vmcnt(0)) before it arrives. A wait that exceeds KT_SPIN_MAX polls sets the status word and gives up;
   once the status is set, later barriers do not wait. Returns false when this block did not wait the barrier out. */
__device__ __forceinline__ bool kt_bar_wait(const unsigned* line0, unsigned n, unsigned want, int lane, unsigned* status){
  for(unsigned it = 0;; ++it){
    const unsigned v = lane < (int)n ? __hip_atomic_load(line0 + lane * KT_BAR_LINE, __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT) : want;
    if(__ballot(v < want) == 0) return true;
    if(it == KT_SPIN_MAX){
      if(lane == 0) __hip_atomic_fetch_or(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
  }
}
__device__ __forceinline__ bool kt_plan_barrier(unsigned* ctr, unsigned k, unsigned G, int lane){
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  unsigned* status = ctr + KT_BAR_STATUS * KT_BAR_LINE;
  const unsigned want = k + 1u, b = blockIdx.x, grp = b / KT_BAR_FAN, ng = (G + KT_BAR_FAN - 1) / KT_BAR_FAN;
  bool ok = __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u;
  if(b % KT_BAR_FAN == 0){
    const unsigned nm = min(G - b, (unsigned)KT_BAR_FAN);          /* the group's blocks, this one included */
    /* lane 0 reads this block's own line, which it has not written: skip it */
    if(ok && nm > 1) ok = kt_bar_wait(ctr + (KT_BAR_ARR + b + 1) * KT_BAR_LINE, nm - 1, want, lane, status);
    if(lane == 0) __hip_atomic_store(ctr + (KT_BAR_GRP + grp) * KT_BAR_LINE, want, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
  } else if(lane == 0)
    __hip_atomic_store(ctr + (KT_BAR_ARR + b) * KT_BAR_LINE, want, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if(ok) ok = kt_bar_wait(ctr + KT_BAR_GRP * KT_BAR_LINE, ng, want, lane, status);
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  return ok;
}

/* the block barrier of the plan: LDS traffic of the wave done, then s_barrier. Unlike __syncthreads it does not
   wait for the wave's global loads and stores (the data waves' prefetch, the control wave's output stores), which
   nothing across this barrier needs: the slice sums meet in LDS, and the stage ordering is the grid barrier's. */
__device__ __forceinline__ void kt_block_sync(){
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

