/* kt_splan.hip - the streamed decode-plan executor (one token): a decode step's products (spec.py:619-673: q/k/v, o,
   gate/up, down, ... of every layer) in one persistent launch whose weight stream runs ahead of the stage ends.

   Work: the row groups of all stages, concatenated in stage order (q = q0[s] + rg), are dealt round-robin to the G
   blocks (block b takes q = b, b + G, ...), so every block carries a near-equal share of every stage. A block's tasks
   of a stage are (row group, K slice) pairs j = i KS + ks; compute wave w takes the tasks with (N + j) % 8 == w (N =
   the block's tasks of earlier stages), so the 8 waves' shares of the step differ by at most one task. A task is
   what k_gemv_flat computes for one slice: lane 8 c + r chains its units 8 st + c of the slice in order
   (fmaf((float)(v - XA), XS * d, .)) and the 8 lane chains are added by the row butterfly; the slice sums meet in
   LDS and are added in slice order when the rows are stored. The same tree, so the same bits as the launches.

   Weights: each compute wave streams its tasks' steps (a step = 8 units of a row group: 2 KB of codes and 128 B of
   scales, contiguous in the kt2 layout) through a ring of KS_D slots in LDS with global_load_lds (DMA: no registers
   held), KS_D steps ahead of the one it computes, across task and stage ends (weights never depend on an earlier
   stage). Every step issues exactly three DMA instructions (stand-ins of the same shape past the wave's last
   task), so "step i is in LDS" is exactly s_waitcnt vmcnt(3 (KS_D - 1)); a compute wave issues no other
   vector-memory instruction, and its LDS accesses are asm so that the compiler adds no waits for the DMA stream.

   Stage ends: a compute wave that has finished its tasks of stage s arrives on an LDS counter and polls the LDS
   stage word. The control wave (the ninth wave, no weight stream) waits for the 8 arrivals, stores the block's rows
   of stage s (agent scope; it waits for them only when a later stage reads them), passes the grid barrier of
   kt_plan.h, loads stage s + 1's activations if they are rows of this launch, publishes stage s + 1, and then DMAs
   stage s + 2's activations into the buffer stage s has released (double-buffered by stage parity). So a stage
   reads only what every earlier stage has completed, as separate launches do.

   Activations in LDS: step st's 8 units at st x 1 KB, unit c's 16-byte chunk i at slot c x 8 + (i ^ c): the chunk
   reads of one instruction (fixed i, 8 units) fall on 8 distinct bank groups. XS / XA of every unit after them. */
#include "kt_plan.h"

#define KS_WB 8                       /* waves a block */
#define KS_D 6                        /* ring slots a wave (steps in flight) */
#define KS_SLOT 2304                  /* a slot: 2 KB of codes, 256 B for the scales */
#define KS_LDS_SPIN (1u << 26)        /* polls of the LDS stage word before a wave gives up (status set) */

#define KT_L3 __attribute__((address_space(3)))
/* s_waitcnt vmcnt(0) expcnt(0) lgkmcnt(0) as the builtin, which the compiler's wait insertion takes into account */
#define KS_WAIT_ALL 0

/* global -> LDS DMA (global_load_lds: lane i's 16 or 4 bytes land at the wave-uniform LDS address + 16 i or 4 i),
   non-temporal (each weight byte is read once a step: the stage table and activations keep their place in L2), in
   asm so that the compiler does not track them: it would otherwise wait for all of them (vmcnt(0)) before LDS
   accesses and register reuse it cannot prove independent. Their completion is waited for explicitly. */
__device__ __forceinline__ void ks_dma16(const void* g, uint8_t* l){
  const unsigned m = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(const KT_L3 void*)l);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off nt" :: "s"(m), "v"(g) : "m0");
}
__device__ __forceinline__ void ks_dma4(const void* g, uint8_t* l){
  const unsigned m = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(const KT_L3 void*)l);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off nt" :: "s"(m), "v"(g) : "m0");
}

/* plan fields through the scalar cache: the stage table is read-only during the launch, but the compiler cannot
   see that across the barrier's atomics and waits and would read it with vector loads, which wait behind the DMA
   stream (vmcnt is in order). Loads only. */
__device__ __forceinline__ int ks_s32(const void* p){
  int v;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p));
  return v;
}
__device__ __forceinline__ const void* ks_s64(const void* p){
  const void* v;
  asm volatile("s_load_dwordx2 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p));
  return v;
}
__device__ __forceinline__ const uint8_t* ks_stage(const uint8_t* plan, int s){
  return plan + KT_PLAN_HDR + (size_t)s * sizeof(KtPStage);
}
#define KS_F(st, field) (ks_s32((st) + offsetof(KtPStage, field)))
#define KS_MF(st, i, field) (ks_s32((st) + offsetof(KtPStage, mat) + (i) * sizeof(KtMat) + offsetof(KtMat, field)))
#define KS_MP(st, i, field) (ks_s64((st) + offsetof(KtPStage, mat) + (i) * sizeof(KtMat) + offsetof(KtMat, field)))
#define KS_F64(st, field) (ks_s64((st) + offsetof(KtPStage, field)))

/* a stage's fields for the weight stream, in one batch of scalar loads and one wait. q1 = the next stage's first row
   group (read from the next record; the caller replaces it for the last stage: the record past the table is still
   inside the plan buffer) */
struct KsSt {
  int q0, q1, KS, NU, nmat, rg1, rg2;
  const uint4* cd0; const uint4* cd1; const uint4* cd2;
  const uint16_t* sc0; const uint16_t* sc1; const uint16_t* sc2;
};
#define KS_OM(i, f) (offsetof(KtPStage, mat) + (i) * sizeof(KtMat) + offsetof(KtMat, f))
__device__ __forceinline__ KsSt ks_ld_stage(const uint8_t* plan, int s, int nS, int qtot){
  KsSt t;
  const uint8_t* p = ks_stage(plan, s);
  asm volatile("s_load_dword %0, %13, %14\n\t"
               "s_load_dword %1, %13, %15\n\t"
               "s_load_dword %2, %13, %16\n\t"
               "s_load_dword %3, %13, %17\n\t"
               "s_load_dword %4, %13, %18\n\t"
               "s_load_dword %5, %13, %19\n\t"
               "s_load_dword %6, %13, %20\n\t"
               "s_load_dwordx2 %7, %13, %21\n\t"
               "s_load_dwordx2 %8, %13, %22\n\t"
               "s_load_dwordx2 %9, %13, %23\n\t"
               "s_load_dwordx2 %10, %13, %24\n\t"
               "s_load_dwordx2 %11, %13, %25\n\t"
               "s_load_dwordx2 %12, %13, %26\n\t"
               "s_waitcnt lgkmcnt(0)"
               : "=&s"(t.q0), "=&s"(t.q1), "=&s"(t.KS), "=&s"(t.NU), "=&s"(t.nmat), "=&s"(t.rg1), "=&s"(t.rg2),
                 "=&s"(t.cd0), "=&s"(t.cd1), "=&s"(t.cd2), "=&s"(t.sc0), "=&s"(t.sc1), "=&s"(t.sc2)
               : "s"(p), "n"(offsetof(KtPStage, q0)), "n"(sizeof(KtPStage) + offsetof(KtPStage, q0)),
                 "n"(offsetof(KtPStage, KS)), "n"(offsetof(KtPStage, NU)), "n"(offsetof(KtPStage, nmat)),
                 "n"(KS_OM(1, rg0)), "n"(KS_OM(2, rg0)), "n"(KS_OM(0, codes)), "n"(KS_OM(1, codes)),
                 "n"(KS_OM(2, codes)), "n"(KS_OM(0, scales)), "n"(KS_OM(1, scales)), "n"(KS_OM(2, scales)));
  if(s + 1 >= nS) t.q1 = qtot;
  if(t.nmat < 2) t.rg1 = 1 << 30;
  if(t.nmat < 3) t.rg2 = 1 << 30;
  return t;
}
/* a wave-uniform value through readfirstlane: a select between such values stays a select of registers (a select
   between fields of a struct would become a load through a selected address, which keeps the struct in scratch) */
__device__ __forceinline__ int ks_u(int v){ return __builtin_amdgcn_readfirstlane(v); }
template <typename T>
__device__ __forceinline__ T* ks_up(T* p){
  const unsigned long long a = (unsigned long long)p;
  return (T*)(((unsigned long long)(unsigned)__builtin_amdgcn_readfirstlane((int)(a >> 32)) << 32)
              | (unsigned)__builtin_amdgcn_readfirstlane((int)a));
}

/* a stage's outputs (rows and counts of its matrices), in one batch */
struct KsOut {
  float* y0; float* y1; float* y2;
  int R0, R1, R2;
};
__device__ __forceinline__ KsOut ks_ld_out(const uint8_t* plan, int s){
  KsOut o;
  const uint8_t* p = ks_stage(plan, s);
  asm volatile("s_load_dwordx2 %0, %6, %7\n\t"
               "s_load_dwordx2 %1, %6, %8\n\t"
               "s_load_dwordx2 %2, %6, %9\n\t"
               "s_load_dword %3, %6, %10\n\t"
               "s_load_dword %4, %6, %11\n\t"
               "s_load_dword %5, %6, %12\n\t"
               "s_waitcnt lgkmcnt(0)"
               : "=&s"(o.y0), "=&s"(o.y1), "=&s"(o.y2), "=&s"(o.R0), "=&s"(o.R1), "=&s"(o.R2)
               : "s"(p), "n"(KS_OM(0, y)), "n"(KS_OM(1, y)), "n"(KS_OM(2, y)), "n"(KS_OM(0, R)), "n"(KS_OM(1, R)),
                 "n"(KS_OM(2, R)));
  return o;
}

/* LDS accesses of a computing wave, in asm: the compiler cannot tell a ring slot being read from the slots whose DMA
   is still in flight, and before a compiled LDS access it would wait for every outstanding vector-memory operation
   (s_waitcnt vmcnt(0)), which empties the ring. Each helper waits for its own LDS operations (lgkmcnt). */
__device__ __forceinline__ unsigned ks_la(const void* p){ return (unsigned)(uintptr_t)(const KT_L3 void*)p; }

struct KsOps {
  kt_u32x4 c0, c1, x[8];
  unsigned hs, xs, xa;
};
/* one step's operands: the lane's two code words and scale from the ring slot, its unit's 8 activation chunks,
   XS and XA of the unit */
__device__ __forceinline__ void ks_read(KsOps& o, unsigned aw, unsigned ah, const unsigned (&ax)[8], unsigned axs,
                                        unsigned axa){
  asm volatile("ds_read_b128 %0, %13\n\t"
               "ds_read_b128 %1, %13 offset:1024\n\t"
               "ds_read_b128 %2, %14\n\t"
               "ds_read_b128 %3, %15\n\t"
               "ds_read_b128 %4, %16\n\t"
               "ds_read_b128 %5, %17\n\t"
               "ds_read_b128 %6, %18\n\t"
               "ds_read_b128 %7, %19\n\t"
               "ds_read_b128 %8, %20\n\t"
               "ds_read_b128 %9, %21\n\t"
               "ds_read_u16 %10, %22\n\t"
               "ds_read_b32 %11, %23\n\t"
               "ds_read_b32 %12, %24\n\t"
               "s_waitcnt lgkmcnt(0)"
               : "=&v"(o.c0), "=&v"(o.c1), "=&v"(o.x[0]), "=&v"(o.x[1]), "=&v"(o.x[2]), "=&v"(o.x[3]), "=&v"(o.x[4]),
                 "=&v"(o.x[5]), "=&v"(o.x[6]), "=&v"(o.x[7]), "=&v"(o.hs), "=&v"(o.xs), "=&v"(o.xa)
               : "v"(aw), "v"(ax[0]), "v"(ax[1]), "v"(ax[2]), "v"(ax[3]), "v"(ax[4]), "v"(ax[5]), "v"(ax[6]),
                 "v"(ax[7]), "v"(ah), "v"(axs), "v"(axa));
}
__device__ __forceinline__ void ks_write32(unsigned a, unsigned v){
  asm volatile("ds_write_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" :: "v"(a), "v"(v));
}
/* an LDS word that another wave publishes: a compiler barrier too, so that reads of what the word announces are not
   moved before the poll */
__device__ __forceinline__ unsigned ks_read32(unsigned a){
  unsigned v;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
  return v;
}
/* lane 0 adds 1 to an LDS counter; every lane gets the old value */
__device__ __forceinline__ unsigned ks_arrive(unsigned a, int lane){
  unsigned old = 0;
  if(lane == 0) asm volatile("ds_add_rtn_u32 %0, %1, %2\n\ts_waitcnt lgkmcnt(0)" : "=v"(old) : "v"(a), "v"(1u));
  return __builtin_amdgcn_readfirstlane(old);
}

/* the LDS layout of a block */
struct KsLds {
  uint8_t* ring;                      /* [KS_WB][KS_D][KS_SLOT] */
  uint8_t* act[2];                    /* [smax][1024] swizzled, by stage parity */
  float* xs[2];                       /* [numax rounded to 64] */
  int* xa[2];
  float* out;                         /* [tmax][8] the slice sums of the block's tasks of the current stage */
  unsigned* ctl;                      /* [0] arrivals, [1] the published stage, [2] error */
};

__host__ __device__ __forceinline__ int ks_nu64(int numax){ return (numax + 63) / 64 * 64; }
__host__ __device__ __forceinline__ size_t ks_lds_bytes(int smax, int numax, int tmax){
  return (size_t)KS_WB * KS_D * KS_SLOT + 2 * ((size_t)smax * 1024 + (size_t)ks_nu64(numax) * 8) + (size_t)tmax * 32
         + 16;
}

/* the block's first row-group index (k) of the rows q >= q0 (its k-th row group is q = b + k G) */
__device__ __forceinline__ int ks_kfirst(int q0, int b, int G){ return q0 <= b ? 0 : (q0 - b + G - 1) / G; }

/* a stage as the block sees it: its row groups k in [kb, ke), its tasks j in [0, ns) (j = i KS + ks: slice ks of the
   block's i-th row group); wave w takes the tasks with (N + j) % KS_WB == w, N = the block's tasks of the earlier
   stages, so the waves' shares of the step differ by at most one task */
struct KsStage {
  KsSt f;
  int kb, ns, St;
};
__device__ __forceinline__ KsStage ks_stage_info(const uint8_t* plan, int s, int nS, int G, int qtot, int b){
  KsStage t;
  t.f = ks_ld_stage(plan, s, nS, qtot);
  t.kb = ks_kfirst(t.f.q0, b, G);
  t.ns = (ks_kfirst(t.f.q1, b, G) - t.kb) * t.f.KS;
  t.St = kt_steps(t.f.NU);
  return t;
}
__device__ __forceinline__ int ks_jfirst(int N, int w){ return ((w - N) % KS_WB + KS_WB) % KS_WB; }

/* a wave's DMA cursor through its tasks' steps (wave-uniform) */
struct KsCur {
  int s, N, live;                     /* stage, the block's tasks before it, 0 past the wave's last task */
  KsStage t;
  int j, st, st1;                     /* task, step, the slice's end step */
  const uint4* cb;                    /* the task's row group: codes, scales */
  const uint16_t* sb;
};
/* move to the wave's next task at or after task d.j of stage d.s, and set its row group and steps */
__device__ __forceinline__ void ks_cur_task(const uint8_t* plan, int nS, int G, int qtot, int b, int w, KsCur& d){
  while(d.live && d.j >= d.t.ns){
    d.N += d.t.ns;
    if(++d.s == nS){ d.live = 0; break; }
    d.t = ks_stage_info(plan, d.s, nS, G, qtot, b);
    d.j = ks_jfirst(d.N, w);
  }
  if(!d.live) return;
  const KsSt& f = d.t.f;
  const int i = d.j / f.KS, ks = d.j - i * f.KS;
  const int rg = b + (d.t.kb + i) * G - f.q0;
  const int rg1 = ks_u(f.rg1), rg2 = ks_u(f.rg2);
  const bool m2 = rg >= rg2, m1 = rg >= rg1;
  const int lrg = rg - (m2 ? rg2 : m1 ? rg1 : 0);
  const uint4* c0 = ks_up(f.cd0); const uint4* c1 = ks_up(f.cd1); const uint4* c2 = ks_up(f.cd2);
  const uint16_t* s0 = ks_up(f.sc0); const uint16_t* s1 = ks_up(f.sc1); const uint16_t* s2 = ks_up(f.sc2);
  d.cb = (m2 ? c2 : m1 ? c1 : c0) + (long long)lrg * f.NU * 16;
  d.sb = (m2 ? s2 : m1 ? s1 : s0) + (long long)lrg * f.NU * 8;
  d.st = ks * d.t.St / f.KS;
  d.st1 = (ks + 1) * d.t.St / f.KS;
}

/* the three DMA instructions of one step (or their stand-ins past the last task) into a ring slot */
__device__ __forceinline__ void ks_issue(const uint8_t* plan, int nS, int G, int qtot, int b, int w, int lane,
                                         KsCur& d, uint8_t* slot){
  const uint8_t* g0 = plan + lane * 16;                            /* stand-ins: 1 KB of the plan header region */
  const uint8_t* g1 = g0;
  const uint8_t* gs = plan + lane * 4;
  if(d.live){
    const int st = d.st, NU = d.t.f.NU, nc = NU - st * KT_KL < KT_KL ? NU - st * KT_KL : KT_KL;
    const uint4* base = d.cb + (long long)st * 128;
    const bool ok = lane < nc * 8;                                 /* lanes past a ragged step read its start */
    g0 = (const uint8_t*)(base + (ok ? lane : 0));
    g1 = (const uint8_t*)(base + (ok ? nc * 8 + lane : 0));
    gs = (const uint8_t*)(d.sb + st * 64) + (lane * 2 < nc * 8 ? lane * 4 : 0);
    if(++d.st == d.st1){
      d.j += KS_WB;
      ks_cur_task(plan, nS, G, qtot, b, w, d);
    }
  }
  ks_dma16(g0, slot);
  ks_dma16(g1, slot + 1024);
  ks_dma4(gs, slot + 2048);
}

/* stage s's activations (token 0) into activation buffer p by one wave: DMA, or coherent loads when an earlier stage
   wrote them. The caller waits for them. */
__device__ __forceinline__ void ks_stage_act(const uint8_t* plan, int s, const KsLds& L, int p, int lane){
  const uint8_t* Sp = ks_stage(plan, s);
  const int NU = KS_F(Sp, NU), St = kt_steps(NU), C = NU * 128, coh = KS_F(Sp, coh);
  const int8_t* xq = (const int8_t*)KS_F64(Sp, xq);
  const float* xs = (const float*)KS_F64(Sp, xs);
  const int* xa = (const int*)KS_F64(Sp, xa);
  const int c = lane >> 3, ip = lane & 7, i = ip ^ c;             /* slot c 8 + ip holds chunk i = ip ^ c of unit c */
  if(!coh){
    for(int st = 0; st < St; ++st){
      const int off = st * 1024 + c * 128 + i * 16;
      ks_dma16(xq + (off < C ? off : 0), (p ? L.act[1] : L.act[0]) + st * 1024);
    }
    for(int u0 = 0; u0 < NU; u0 += 64){
      const int u = u0 + lane < NU ? u0 + lane : 0;
      ks_dma4(xs + u, (uint8_t*)((p ? L.xs[1] : L.xs[0]) + u0));
      ks_dma4(xa + u, (uint8_t*)((p ? L.xa[1] : L.xa[0]) + u0));
    }
  } else {
    for(int st = 0; st < St; ++st){
      const int off = st * 1024 + c * 128 + i * 16;
      const KT_G unsigned* q4 = (const KT_G unsigned*)(xq + (off < C ? off : 0));
      uint4 v;
      v.x = __hip_atomic_load(q4, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      v.y = __hip_atomic_load(q4 + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      v.z = __hip_atomic_load(q4 + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      v.w = __hip_atomic_load(q4 + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *(uint4*)((p ? L.act[1] : L.act[0]) + st * 1024 + lane * 16) = v;
    }
    for(int u = lane; u < NU; u += 64){
      (p ? L.xs[1] : L.xs[0])[u] = __uint_as_float(__hip_atomic_load((const KT_G unsigned*)(xs + u), __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT));
      (p ? L.xa[1] : L.xa[0])[u] = (int)__hip_atomic_load((const KT_G unsigned*)(xa + u), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

/* the exact value of a unit from its two code words and its 8 activation chunks (as kt_unit_lds) */
__device__ __forceinline__ int ks_unit(const kt_u32x4 c0, const kt_u32x4 c1, const kt_u32x4 (&xc)[8]){
  int a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
  for(int h = 0; h < 2; ++h){
    const kt_u32x4 cw = h ? c1 : c0;
    const uint32_t ww[4] = {cw.x, cw.y, cw.z, cw.w};
#pragma unroll
    for(int j = 0; j < 4; ++j){
      const kt_u32x4 x = xc[4 * h + j];
      a0 = kt_dot4((int)(ww[j] & 0x03030303u), (int)x.x, a0);
      a1 = kt_dot4((int)(ww[j] & 0x0C0C0C0Cu), (int)x.y, a1);
      a2 = kt_dot4((int)(ww[j] & 0x30303030u), (int)x.z, a2);
      a0 = kt_dot4((int)((ww[j] >> 6) & 0x03030303u), (int)x.w, a0);
    }
  }
  return a0 + (a1 >> 2) + (a2 >> 4);
}

/* the block's rows of stage s: row r of its i-th row group = the slice sums of the row in slice order (the tree of
   the single launches), stored with agent scope (lane = 8 i' + r over groups of 8 row groups) */
__device__ __forceinline__ void ks_store_rows(const uint8_t* plan, int s, const KsStage& t, int b, int G,
                                              const KsLds& L, int lane){
  const KsOut m = ks_ld_out(plan, s);
  const int nr = t.ns / t.f.KS, KS = t.f.KS;
  const int c = lane >> 3, r = lane & 7;
  for(int i0 = 0; i0 < nr; i0 += 8){
    const int i = i0 + c;
    if(i < nr){
      const int rg = b + (t.kb + i) * G - t.f.q0;
      const int rg1 = ks_u(t.f.rg1), rg2 = ks_u(t.f.rg2);
      const bool m2 = rg >= rg2, m1 = rg >= rg1;
      float* y = m2 ? ks_up(m.y2) : m1 ? ks_up(m.y1) : ks_up(m.y0);
      const int R = m2 ? ks_u(m.R2) : m1 ? ks_u(m.R1) : ks_u(m.R0), rgm = m2 ? rg2 : m1 ? rg1 : 0;
      const int row = (rg - rgm) * KT_RG + r;
      float v = L.out[(i * KS) * 8 + r];
      for(int ks = 1; ks < KS; ++ks) v += L.out[(i * KS + ks) * 8 + r];
      if(row < R) __hip_atomic_store((KT_G float*)(y + row), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

__global__ void __launch_bounds__(64 * (KS_WB + 1)) k_splan(const uint8_t* __restrict__ plan,
                                                             unsigned* __restrict__ ctr){
  extern __shared__ __attribute__((aligned(16))) uint8_t kt_lds[];
  const int nS = ks_s32(plan + offsetof(KtPlanHdr, nstages)), G = ks_s32(plan + offsetof(KtPlanHdr, G));
  const int smax = ks_s32(plan + offsetof(KtPlanHdr, smax)), numax = ks_s32(plan + offsetof(KtPlanHdr, numax));
  const int tmax = ks_s32(plan + offsetof(KtPlanHdr, tmax)), qtot = ks_s32(plan + offsetof(KtPlanHdr, qtot));
  const int b = blockIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, c = lane >> 3, r = lane & 7;
  KsLds L;
  L.ring = kt_lds;
  uint8_t* q = L.ring + KS_WB * KS_D * KS_SLOT;
  for(int p = 0; p < 2; ++p){
    L.act[p] = q;
    L.xs[p] = (float*)(q + (size_t)smax * 1024);
    L.xa[p] = (int*)(L.xs[p] + ks_nu64(numax));
    q = (uint8_t*)(L.xa[p] + ks_nu64(numax));
  }
  L.out = (float*)q;
  L.ctl = (unsigned*)(L.out + (size_t)tmax * 8);

  if(w == KS_WB){
    /* ---------------------------------------------------------------- control wave (no weight stream) */
    if(lane == 0){ L.ctl[0] = 0u; L.ctl[1] = 0u; L.ctl[2] = 0u; }
    ks_stage_act(plan, 0, L, 0, lane);
    if(nS > 1 && !KS_F(ks_stage(plan, 1), coh)) ks_stage_act(plan, 1, L, 1, lane);
    __builtin_amdgcn_s_waitcnt(KS_WAIT_ALL);
    kt_block_sync();
    KsStage tc = ks_stage_info(plan, 0, nS, G, qtot, b);
    for(int s = 0; s < nS; ++s){
      /* the flags this stage end needs, read while the compute waves work */
      const int pub = KS_F(ks_stage(plan, s), pub);
      const int coh1 = s + 1 < nS ? KS_F(ks_stage(plan, s + 1), coh) : 0;
      const int coh2 = s + 2 < nS ? KS_F(ks_stage(plan, s + 2), coh) : 1;
      unsigned n = 0;                                              /* every compute wave has finished stage s */
      while(__builtin_amdgcn_readfirstlane(ks_read32(ks_la(L.ctl))) < (unsigned)(KS_WB * (s + 1))){
        __builtin_amdgcn_s_sleep(1);
        if(++n == KS_LDS_SPIN){ if(lane == 0) ks_write32(ks_la(L.ctl + 2), 1u); break; }
      }
      const KsStage t = tc;
      ks_store_rows(plan, s, t, b, G, L, lane);
      if(pub) __builtin_amdgcn_s_waitcnt(KS_WAIT_ALL);              /* read by a later stage: stored first */
      if(s + 1 < nS){
        kt_plan_barrier(ctr, (unsigned)s, (unsigned)G, lane);
        if(coh1){                                                   /* reads what an earlier stage wrote */
          ks_stage_act(plan, s + 1, L, (s + 1) & 1, lane);
          __builtin_amdgcn_s_waitcnt(KS_WAIT_ALL);
        }
        if(lane == 0) ks_write32(ks_la(L.ctl + 1), (unsigned)(s + 1));
        /* stage s + 2's activations into the buffer stage s has released (unless it reads this launch's rows) */
        if(!coh2){
          ks_stage_act(plan, s + 2, L, s & 1, lane);
          __builtin_amdgcn_s_waitcnt(KS_WAIT_ALL);
        }
      }
      if(s + 1 < nS) tc = ks_stage_info(plan, s + 1, nS, G, qtot, b);   /* off the stage-end path */
    }
    if(L.ctl[2] && lane == 0) __hip_atomic_fetch_or(ctr + KT_BAR_STATUS * KT_BAR_LINE, 2u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
    return;
  }

  /* ------------------------------------------------------------------ compute wave w: the first KS_D steps */
  uint8_t* ring = L.ring + (size_t)w * KS_D * KS_SLOT;
  KsCur d;
  d.s = 0; d.N = 0; d.live = nS > 0 ? 1 : 0;
  d.t = ks_stage_info(plan, 0, nS, G, qtot, b);
  d.j = ks_jfirst(0, w);
  d.st = d.st1 = 0; d.cb = nullptr; d.sb = nullptr;
  ks_cur_task(plan, nS, G, qtot, b, w, d);
  for(int i = 0; i < KS_D; ++i) ks_issue(plan, nS, G, qtot, b, w, lane, d, ring + i * KS_SLOT);
  kt_block_sync();

  int cnt = 0, N = 0;                                               /* steps computed; the block's earlier tasks */
  KsStage tn = ks_stage_info(plan, 0, nS, G, qtot, b);
  for(int s = 0; s < nS; ++s){
    const KsStage t = tn;
    if(s + 1 < nS) tn = ks_stage_info(plan, s + 1, nS, G, qtot, b);   /* read before the wait, not after */
    if(s > 0){
      unsigned n = 0;
      while(__builtin_amdgcn_readfirstlane(ks_read32(ks_la(L.ctl + 1))) < (unsigned)s){
        __builtin_amdgcn_s_sleep(1);
        if(++n == KS_LDS_SPIN){ if(lane == 0) ks_write32(ks_la(L.ctl + 2), 1u); break; }
      }
    }
    const int p = s & 1, NU = t.f.NU, St = t.St, KS = t.f.KS;
    for(int j = ks_jfirst(N, w); j < t.ns; j += KS_WB){
      const int i = j / KS, ks = j - i * KS;
      float chain = 0.0f;
      for(int st = ks * St / KS; st < (ks + 1) * St / KS; ++st){
        uint8_t* slot = ring + (cnt % KS_D) * KS_SLOT;
        const int nc = NU - st * KT_KL < KT_KL ? NU - st * KT_KL : KT_KL;
        const int u = st * KT_KL + c;
        const bool uok = c < nc;
        const int uu = uok ? u : 0;
        unsigned ax[8];
        const unsigned a0 = ks_la((p ? L.act[1] : L.act[0]) + st * 1024 + c * 128);
#pragma unroll
        for(int x = 0; x < 8; ++x) ax[x] = a0 + ((x ^ c) << 4);
        KsOps o;
        asm volatile("s_waitcnt vmcnt(%0)" :: "n"(3 * (KS_D - 1)) : "memory");
        ks_read(o, ks_la(slot + lane * 16), ks_la(slot + 2048 + lane * 2), ax, ks_la((p ? L.xs[1] : L.xs[0]) + uu),
                ks_la((p ? L.xa[1] : L.xa[0]) + uu));
        int v = ks_unit(o.c0, o.c1, o.x) - (int)o.xa;
        v = uok ? v : 0;
        const float dsc = uok ? kt_h2f((uint16_t)o.hs) : 0.0f;
        chain = fmaf((float)v, __uint_as_float(o.xs) * dsc, chain);
        ks_issue(plan, nS, G, qtot, b, w, lane, d, slot);
        ++cnt;
      }
      const float y = kt_row_sum(chain);
      if(c == 0) ks_write32(ks_la(L.out + j * 8 + r), __float_as_uint(y));
    }
    N += t.ns;
    ks_arrive(ks_la(L.ctl), lane);                                  /* after the slice sums (LDS is in order) */
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");                 /* the stand-in DMAs of the stream's tail */
}

size_t kt_splan_lds(int smax, int numax, int tmax){ return ks_lds_bytes(smax, numax, tmax); }
const void* kt_splan_kernel(){ return (const void*)k_splan; }
