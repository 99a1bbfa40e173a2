/* kt_api.hip - the C ABI of libkt_gfx950.so: host-side validation and launches. Every entry point takes
   caller-owned device pointers and a stream (NULL = the null stream), never allocates, never synchronizes, and
   returns a hipError_t as int (0 = success; hipErrorInvalidValue for shapes or strides the kernels do not take).
   The declarations and the reference interfaces they replace are in include/kt.h. */
#include "kt_common.h"
#include <vector>
#include <algorithm>
#include <mutex>
#include "../../include/kt.h"
#include "kt_fold.h"
#include "kt_launch.h"
#include "kt_topk.h"

template <int FMT, int MT, bool DBG, bool GRP>
__global__ void k_gemv_flat(const KtGemvArgs, const KtGroupedArgs, const int8_t*, const float*, const int*, int32_t*,
                            int);
template <int FMT, int MT, bool DBG, bool GRP>
__global__ void k_gemv_flat1(const KtGemvArgs, const KtGroupedArgs, const int8_t*, const float*, const int*, int32_t*,
                             int);
template <int RG, bool DBG>
__global__ void k_gemv_step(const KtGemvArgs, const int8_t*, const float*, const int*, int32_t*, int);
template <int MT, bool DBG>
__global__ void k_gemv_stepm(const KtGemvArgs a, const int8_t* __restrict__ xq, const float* __restrict__ xs,
                             const int* __restrict__ xa, int32_t* __restrict__ dbg, int KS);
template <bool DBG>
__global__ void k_gemv_pair(const KtGemvArgs, const int8_t*, const float*, const int*, int32_t*, int);
template <int NT, bool DBG, int LB>
__global__ void k_gemv_mma(const KtGemvArgs, const int8_t*, const float*, int32_t*, int);
template <bool DBG, int KQ, bool MS>
__global__ void k_gemv_m16(const KtGemvArgs, const int8_t*, const float*, const int*, int32_t*, int);
template <bool GRP, bool DBG, bool MS>
__global__ void k_q8_mma(const KtGemvArgs, const KtGroupedArgs, const int8_t*, const float*, int32_t*, int);
template <int SRC> __global__ void k_tern_pack(const uint8_t*, const uint16_t*, int, int, uint32_t*, uint16_t*);
extern "C" __global__ void k_q8_pack(const uint8_t*, int, int, uint32_t*, uint16_t*);
extern "C" __global__ void k_tern_pack_ptq1(const uint8_t*, int, int, int, int, uint32_t*, uint16_t*);
extern "C" __global__ void k_quant_tern(const float*, int, int, int, int8_t*, int, float*, int*);
extern "C" __global__ void k_quant_q8(const float*, int, int, int, int8_t*, int, float*, int);
extern "C" __global__ void k_tern_sum(const float*, float*, int, int, int);
template <bool DBG, bool RS>
__global__ void k_tern_gemm(const uint32_t*, const uint16_t*, int, int, const int8_t*, int, const float*, int, float*,
                            uint16_t*, int, int32_t*);
extern "C" __global__ void k_tern_expand(const uint4*, int, long long, int, int8_t*);
template <bool DBG>
__global__ void k_tern_gemm8(const int8_t*, const uint16_t*, int, int, const int8_t*, int, const float*, int, float*,
                             uint16_t*, int, int32_t*, int, int);
size_t kt_gemm8_lds();
template <int WT, int WR, int PD, bool DBG>
__global__ void k_tern_gemm_rs1(const uint32_t*, const uint16_t*, int, int, const int8_t*, int, const float*, int,
                                float*, uint16_t*, int, int32_t*);
__global__ void k_moe_topk(const float*, int, int, const KtRouter, int*, float*);
extern "C" __global__ void k_moe_sort(const int*, int, int, int*, int*, int*, int*, int*, int*, int);
extern "C" __global__ void k_moe_combine(const float*, const float*, const int*, const float*, int, int, float*, int);
__global__ void k_moe_route(const float*, int, int, int, const KtRouter, int*, float*, int*, int*, int*, int*, int*,
                            int*, const float*, int, int, int8_t*, int, float*, int);
__global__ void k_moe1_up(const float*, int, int, const KtRouter, const uint8_t* const*, const uint8_t* const*, int,
                          int, const float*, float*, int*, float*, const uint8_t**, int);
__global__ void k_moe1_down(const uint8_t* const*, const float*, int, int, int, const float*, float*, float*,
                            const float*, int);
size_t kt_moe1_up_lds(int KS);
size_t kt_moe1_down_lds(int k, int KS);

#define KT_INVALID ((int)hipErrorInvalidValue)
#ifndef KT_STEPM_WAVES
#define KT_STEPM_WAVES 2048           /* multi-token grids of at most this many one-step waves take k_gemv_stepm */
#endif
#ifndef KT_M16H_WAVES
#define KT_M16H_WAVES 16384           /* ... and above 8 tokens, 2 waves a slice on grids of at most this many */
#endif
#ifndef KT_M16Q_MSM
#define KT_M16Q_MSM 8                 /* ... above 4 slices at up to this many tokens */
#endif
#ifndef KT_M16Q_WAVES
#define KT_M16Q_WAVES 16384           /* matrix-core grids of at most this many waves split a slice over 4 waves */
#endif
#ifndef KT_STEP2_WAVES
#define KT_STEP2_WAVES (1ll << 40)    /* one-token k_gemv_step grids of more slice-waves: two row groups a block (never) */
#endif
#ifndef KT_PAIR_WAVES
#define KT_PAIR_WAVES 6144             /* one-token grids of more waves take two row groups a block (k_gemv_pair) */
#endif
#define KT_RS_BLOCKS 1024              /* per-row prefill on small blocks while the 128 x 128 grid has fewer blocks */

static inline hipStream_t kt_stream(void* s){ return (hipStream_t)s; }
static inline bool kt_al(const void* p, size_t a){ return ((uintptr_t)p % a) == 0; }
/* bytes of a matrix's codes and scales (both layouts: 32 bytes and one fp16 per row and unit, rows padded to 8) */
static inline size_t kt_code_bytes(int R, int NU){ return (size_t)kt_r8(R) * NU * 256; }
static inline size_t kt_scale_bytes(int R, int NU){ return (size_t)kt_r8(R) * NU * 16; }
/* K slices of a decode product: a function of the step count S = ceil(units / 8) only (never of M or R), so a
   token's result does not depend on how many tokens share the pass, and a matrix gives the same bits alone or in a
   multi-matrix launch: slices of at most KT_SL steps, at most KT_KSMAX of them */
static int kt_kslices(int NU){
  const int S = kt_steps(NU), ks = (S + KT_SL - 1) / KT_SL;
  return ks < KT_KSMAX ? ks : KT_KSMAX;
}

/* up to 32 ternary tokens: the matrix-core product (the same numbers and tree, so the same bits), tiles of 32 rows
   of one matrix, passes of 16 tokens, on every launch from 3 tokens (measured on MI355X with k_gemv_m16 and its
   k-lanes split over 4 waves on small grids, per launch over 16 27B-class layers and per 2B-class layer: 27B layer
   at 3 / 5 / 7 tokens 56.1 / 81.1 / 50.5 -> 46.6 / 47.8 / 49.6 us, 2B layer 18.8 / 26.0 / 27.4 -> 18.7 / 19.1 /
   19.9 us against the v_dot4 kernels or the earlier size rule). At 2 tokens only launches of 2^26 weights or more
   (27B gate/up 17.7 -> 16.8 us, down 13.8 -> 12.6 us; the 27B layer 43.5 -> 41.6 us); the smaller ones stay faster
   on v_dot4 (27B q/k/v 6.39 against 6.52 us, 2B layer 13.6 against 16.9 us) */
#ifndef KT_MMA_MIN
#define KT_MMA_MIN 3
#endif
#define KT_Q8_MMA_MIN 12               /* q8_0 dense: the matrix-core product from 12 tokens */
#define KT_MMA_MAX 32
#define KT_Q8_MMA_KS 8                 /* q8_0 matrix-core product: K slices a block (kt_mma.hip KM_Q8_KS) */
#ifndef KT_MMA_W2
#define KT_MMA_W2 (1ll << 26)          /* 2 tokens: the matrix cores from this many weights a launch */
#endif
static bool kt_use_mma(const KtGemvArgs& a){
  if(a.M > KT_MMA_MAX || (long long)a.M * a.ldq >= (1ll << 30)) return false;
  if(a.M >= KT_MMA_MIN) return true;
  if(a.M < 2) return false;
  long long w = 0;
  for(int i = 0; i < a.nmat; ++i) w += (long long)a.mat[i].R * a.NU * 128;
  return w >= KT_MMA_W2;
}

static int kt_launch_mma(KtGemvArgs a, const int8_t* xq, const float* xs, const int* xa, int32_t* dbg,
                         hipStream_t s){
  const int ks = kt_kslices(a.NU);
  int tiles = 0;
  for(int i = 0; i < a.nmat; ++i){ a.mat[i].pad = tiles; tiles += (kt_r8(a.mat[i].R) + 3) / 4; }
  const dim3 grid(tiles, (a.M + 15) / 16), block(64 * ks);
  const size_t lds = (size_t)ks * 16 * 32 * 4 + (size_t)ks * 256 * 4;        /* slice sums, XS */
  bool off32 = (long long)a.M * a.ldxs * 4 < (1ll << 31);      /* k_gemv_m16 reads through 32-bit buffer offsets */
  for(int i = 0; i < a.nmat; ++i) off32 = off32 && kt_code_bytes(a.mat[i].R, a.NU) < (1ull << 31);
  if(ks <= 10 && off32){
    /* 16x16x64 tiles for every matrix-core launch up to 10 slices (measured on MI355X: 27B-class step at 16 tokens
       4.10 -> 3.99 ms; 2B-class layer at 8 tokens 27.26 -> 27.03 us, at 6 and 7 tokens even; 27B-class launches at
       6 tokens q/k/v 8.72 -> 8.38, gate/up 22.04 -> 19.51, down 16.14 -> 14.62 us) */
    const bool ms = ks > 4;                                                 /* more slices than 4 groups */
    const int G = ms ? 4 : ks;                                              /* slice groups of the split */
    const long long waves4 = (long long)tiles * grid.y * G * 4;
    if(waves4 <= KT_M16Q_WAVES && (!ms || a.M <= KT_M16Q_MSM)){
      /* the k-lanes of a slice over 4 waves (measured on MI355X against whole-slice waves: 27B-class step at 16
         tokens 3.85 -> 3.71 ms, q/k/v 8.5 -> 7.9 us, gate/up 25.3 -> 24.7 us; 27B-class layer at 3 tokens 47.6 -> 44.1
         us; 2B-class layer at 8 tokens 27.0 -> 18.0 us; a cap of 4096 or 8192 split waves, which left gate/up whole,
         was slower). Above 4 slices a wave takes up to ceil(KS / 4) slices (the 27B down launch at 3 / 5 / 8 tokens
         13.8 / 14.2 / 15.0 -> 12.8 / 13.0 / 14.2 us; slower at 16 tokens, 17.35 -> 17.75 us, so up to 8 tokens) */
      const size_t lq = (size_t)ks * 4 * 16 * 32 * 4 + (size_t)G * 4 * 512 * 4;   /* pair sums, XS + XA a wave */
      const dim3 bq(256 * G);
      if(ms){
        if(dbg) KT_LAUNCH((k_gemv_m16<true, 4, true>), grid, bq, lq, s, a, xq, xs, xa, dbg, ks);
        else KT_LAUNCH((k_gemv_m16<false, 4, true>), grid, bq, lq, s, a, xq, xs, xa, dbg, ks);
      } else {
        if(dbg) KT_LAUNCH((k_gemv_m16<true, 4, false>), grid, bq, lq, s, a, xq, xs, xa, dbg, ks);
        else KT_LAUNCH((k_gemv_m16<false, 4, false>), grid, bq, lq, s, a, xq, xs, xa, dbg, ks);
      }
    } else if(ks > 4 && a.M > KT_M16Q_MSM && (long long)tiles * grid.y * 16 <= KT_M16H_WAVES){
      /* above 8 tokens: the k-lanes of a slice over 2 waves, 8 slice groups (16 waves a block; measured on MI355X,
         27B-class down at 16 tokens 17.41 -> 17.19 us against whole-slice waves) */
      const size_t lh = (size_t)ks * 2 * 16 * 32 * 4 + (size_t)16 * 512 * 4;
      if(dbg) KT_LAUNCH((k_gemv_m16<true, 2, true>), grid, dim3(1024), lh, s, a, xq, xs, xa, dbg, ks);
      else KT_LAUNCH((k_gemv_m16<false, 2, true>), grid, dim3(1024), lh, s, a, xq, xs, xa, dbg, ks);
    } else {
      const size_t lds16 = lds + (size_t)ks * 256 * 4;                      /* + XA */
      if(dbg) KT_LAUNCH((k_gemv_m16<true, 1, false>), grid, block, lds16, s, a, xq, xs, xa, dbg, ks);
      else KT_LAUNCH((k_gemv_m16<false, 1, false>), grid, block, lds16, s, a, xq, xs, xa, dbg, ks);
    }
  } else {
    /* above 10 slices, or buffers past 32-bit offsets: 32x32x32 tiles, the 1024-thread bound (activations loaded in
       place, 124 VGPRs) */
    if(dbg) KT_LAUNCH((k_gemv_mma<16, true, 64 * KT_KSMAX>), grid, block, lds, s, a, xq, xs, dbg, ks);
    else KT_LAUNCH((k_gemv_mma<16, false, 64 * KT_KSMAX>), grid, block, lds, s, a, xq, xs, dbg, ks);
  }
  return 0;
}

/* one block per row group, every token in the launch (chunks of MT tokens whose staging fits in 64 KB of LDS) */
template <int FMT>
static int kt_launch_gemv(const KtGemvArgs& a, int ngroups, const int8_t* xq, const float* xs, const int* xa,
                          int32_t* dbg, hipStream_t s){
  if(FMT == KT_FMT_TERN && kt_use_mma(a)) return kt_launch_mma(a, xq, xs, xa, dbg, s);
  const int ks = kt_kslices(a.NU);
  bool even = true;
  for(int i = 0; i < a.nmat; ++i) even = even && kt_r8(a.mat[i].R) % 2 == 0;
  if(FMT == KT_FMT_TERN && a.M == 1 && kt_steps(a.NU) <= 8){
    /* one step a wave (rows of up to 8 steps, the same tree; measured on MI355X, 27B-class one-token launches against
       two steps a wave: gate/up 11.5 -> 10.9 us, q/k/v 5.6 -> 5.1 us, o 5.0 -> 4.7 us; step 1.91 -> 1.81 ms), one
       row group a block: with the activations loaded before the weights, the 27B gate/up grid (21,760 one-step waves,
       more than the wave slots) is faster on one row group a block than on two (step 1.755 -> 1.736 ms), where it
       was slower with the weights first. KT_STEP2_WAVES: grids of more slice-waves take two row groups a block. Wider
       rows (the 27B down projection: 17 steps) stay on k_gemv_flat1: 16-wave blocks of one step each were slower */
    const int S = kt_steps(a.NU);
    const bool two = even && (long long)ngroups * ks > KT_STEP2_WAVES;
    const size_t lds = (size_t)S * KT_KL * KtFlat<KT_FMT_TERN, 1>::UP + (size_t)(two ? 2 : 1) * S * 64 * 4 * 2;
    const dim3 block(64 * S);
#define KT_ST(RG) do { const dim3 grid(ngroups / RG); \
    if(dbg) KT_LAUNCH((k_gemv_step<RG, true>), grid, block, lds, s, a, xq, xs, xa, dbg, ks); \
    else KT_LAUNCH((k_gemv_step<RG, false>), grid, block, lds, s, a, xq, xs, xa, dbg, ks); } while(0)
    if(two) KT_ST(2); else KT_ST(1);
#undef KT_ST
    return 0;
  }
  if(FMT == KT_FMT_TERN && a.M > 1 && kt_steps(a.NU) <= 8 && (long long)ngroups * kt_steps(a.NU) <= KT_STEPM_WAVES){
    /* the tokens below the matrix-core kernels (2, and 3 - 5 where a pass's activation span reaches 2^30 bytes; the
       two-row form included), one step a wave, on grids that leave the CUs short of waves: 8 a CU or fewer once
       split (measured on MI355X, 2B-class launches at 4 tokens against k_gemv_flat: q/k/v 5.40 -> 4.90 us, o 5.21 ->
       4.66 us; the larger gate/up grid was slower split, 5.93 -> 6.25 us, and stays on k_gemv_flat) */
    const int S = kt_steps(a.NU), mt = a.M <= 2 ? 2 : 4;
    const size_t lds = (size_t)S * mt * KT_KL * KtFlat<KT_FMT_TERN, 1>::UP + (size_t)S * mt * 64 * 4 * 2;
    const dim3 grid(ngroups), block(64 * S);
#define KT_STM(MT) do { \
    if(dbg) KT_LAUNCH((k_gemv_stepm<MT, true>), grid, block, lds, s, a, xq, xs, xa, dbg, ks); \
    else KT_LAUNCH((k_gemv_stepm<MT, false>), grid, block, lds, s, a, xq, xs, xa, dbg, ks); } while(0)
    if(mt == 2) KT_STM(2);
    else KT_STM(4);
#undef KT_STM
    return 0;
  }
  if(FMT == KT_FMT_TERN && a.M == 1 && even && (long long)ngroups * ks > KT_PAIR_WAVES && kt_steps(a.NU) <= KT_SL * ks){
    /* one token on a grid too large for the wave slots: two row groups a block, one round of blocks */
    const dim3 grid(ngroups / 2), block(64 * ks);
    const size_t lds = (size_t)ks * KtFlat<KT_FMT_TERN, 1>::XW + (size_t)ks * 2 * 8 * 4;
    if(dbg) KT_LAUNCH((k_gemv_pair<true>), grid, block, lds, s, a, xq, xs, xa, dbg, ks);
    else KT_LAUNCH((k_gemv_pair<false>), grid, block, lds, s, a, xq, xs, xa, dbg, ks);
    return 0;
  }
  int mt = a.M <= 1 ? 1 : a.M <= 2 ? 2 : 4;
  while(mt > 1 && (mt == 4 ? KtFlat<FMT, 4>::lds(ks) : KtFlat<FMT, 2>::lds(ks)) > 65536) mt >>= 1;
  if(a.hp && mt < 2) return KT_INVALID;                      /* a token's two rows share a chunk */
  const dim3 grid(ngroups), block(64 * ks);
  const KtGroupedArgs ga = {};
#define KT_F(K, MT) do { const size_t lds = KtFlat<FMT, MT>::lds(ks); \
    if(dbg) KT_LAUNCH((K<FMT, MT, true, false>), grid, block, lds, s, a, ga, xq, xs, xa, dbg, ks); \
    else KT_LAUNCH((K<FMT, MT, false, false>), grid, block, lds, s, a, ga, xq, xs, xa, dbg, ks); } while(0)
  if(mt == 4) KT_F(k_gemv_flat, 4); else if(mt == 2) KT_F(k_gemv_flat, 2); else KT_F(k_gemv_flat1, 1);
#undef KT_F
  return 0;
}

static int kt_tern_gemv_n(int nmat, const void* const* W, const int* Rs, float* const* Ys, const int* ldys, int C,
                          const int8_t* XQ, int ldq, const float* XS, const int32_t* XA, int M, int32_t* dbg,
                          void* stream){
  /* M | KT_HP: M tokens of two input rows each (kt_quant_q8 per_row 2, the producers' HB | KT_HP) */
  const int hp = (M & KT_HP) ? 1 : 0;
  M &= ~KT_HP;
  if(M == 0) return 0;
  if(hp){
    if(M < 0 || M > (1 << 29)) return KT_INVALID;
    M *= 2;                                                  /* input rows */
  }
  if(M < 0 || C <= 0 || C % 128 || !XQ || !XS || !XA || ldq < C || ldq % 16 || !kt_al(XQ, 16)) return KT_INVALID;
  KtGemvArgs a = {};
  const int NG = C / 128;
  int groups = 0;
  for(int i = 0; i < nmat; ++i){
    if(!W[i] || !Ys[i] || Rs[i] <= 0 || ldys[i] < Rs[i] || !kt_al(W[i], 16)) return KT_INVALID;
    a.mat[i].codes = (const uint32_t*)W[i];
    a.mat[i].scales = (const uint16_t*)((const uint8_t*)W[i] + kt_code_bytes(Rs[i], NG));
    a.mat[i].y = Ys[i];
    a.mat[i].R = Rs[i];
    a.mat[i].ldy = ldys[i];
    a.mat[i].rg0 = groups;
    groups += kt_r8(Rs[i]);
  }
  if(dbg && nmat != 1) return KT_INVALID;
  a.nmat = nmat;
  a.NU = NG;
  a.ldq = ldq;
  a.ldxs = NG;
  a.M = M;
  a.hp = hp;
  return kt_launch_gemv<KT_FMT_TERN>(a, groups, XQ, XS, (const int*)XA, dbg, kt_stream(stream));
}

/* the MoE decode chain (kt_moe_decode): the workspace's sections, 256-byte aligned */
struct KtMoeWork {
  size_t ids, gw, cnt, off, xrow, where, act, nact, pd, u, yd, total;
};
static bool kt_moe_work(int M, int k, int E, int H, int F, KtMoeWork& w){
  if(M <= 0 || k <= 0 || k > 16 || M > 64 || (long long)M * k > 64 || E <= 0 || E > 1024 || k > E || H <= 0 || F <= 0
     || H % 32 || F % 32 || H > (1 << 20) || F > (1 << 20)) return false;
  const size_t n = (size_t)M * k;
  size_t o = 0;
  auto put = [&](size_t bytes){ const size_t at = o; o += (bytes + 255) / 256 * 256; return at; };
  w.ids = put(n * 4); w.gw = put(n * 4); w.cnt = put((size_t)E * 4); w.off = put((size_t)E * 4);
  w.xrow = put(n * 4); w.where = put(n * 4); w.act = put((size_t)E * 4); w.nact = put(4); w.pd = put(n * 8);
  w.u = put(n * F * 4); w.yd = put(n * H * 4);
  w.total = o;
  return true;
}

/* one grouped q8_0 product on the v_dot4 kernel, activations quantized in the staging from fp32 rows (FMT Q8X, Q8R) */
template <int FMT>
static int kt_grouped_xf(const KtGroupedArgs& a, int E, int nentries, int M, hipStream_t s){
  const int ks = kt_kslices(a.NU);
  const int ny = E < nentries ? E : nentries;
  const int mt = M <= 1 ? 1 : 2;
  const dim3 grid(kt_r8(a.R), ny), block(64 * ks);
  const KtGemvArgs da = {};
  const size_t lds1 = KtFlat<FMT, 1>::lds(ks), lds2 = KtFlat<FMT, 2>::lds(ks);
  if(mt == 1)
    KT_LAUNCH((k_gemv_flat1<FMT, 1, false, true>), grid, block, lds1, s, da, a,
                       (const int8_t*)nullptr, (const float*)nullptr, (const int*)nullptr, (int32_t*)nullptr, ks);
  else
    KT_LAUNCH((k_gemv_flat<FMT, 2, false, true>), grid, block, lds2, s, da, a,
                       (const int8_t*)nullptr, (const float*)nullptr, (const int*)nullptr, (int32_t*)nullptr, ks);
  return 0;
}

static int kt_moe_decode_run(const void* const* Wup, const void* const* Wdown, int E, int H, int F, int k,
                             const KtRouter& rt, const float* logits, int M, float* x, int ldx, const float* ysh, uint8_t* work,
                             size_t work_bytes, hipStream_t s){
  KtMoeWork w;
  if(!kt_moe_work(M, k, E, H, F, w) || !Wup || !Wdown || !logits || !x || !work || ldx < H || ldx % 4
     || !kt_al(x, 16) || !kt_al(work, 256) || work_bytes < w.total) return KT_INVALID;
  int* ids = (int*)(work + w.ids); float* gw = (float*)(work + w.gw);
  int* cnt = (int*)(work + w.cnt); int* off = (int*)(work + w.off); int* xrow = (int*)(work + w.xrow);
  int* where = (int*)(work + w.where); int* act = (int*)(work + w.act); int* nact = (int*)(work + w.nact);
  float* u = (float*)(work + w.u); float* yd = (float*)(work + w.yd);
  const int ksu = kt_kslices(H / 32), ksd = kt_kslices(F / 32);
  if(M == 1 && k <= 8 && ksu <= 16 && ksd * ((k + 1) / 2) <= 16 && kt_steps(F / 32) <= 2 * ksd
     && kt_steps(H / 32) <= 2 * ksu){
    /* one token: the up launch routes for itself; the down launch takes all k picks of a row group and combines */
    const uint8_t* const* wu = (const uint8_t* const*)Wup;
    const uint8_t* const* wd = (const uint8_t* const*)Wdown;
    const uint8_t** pd = (const uint8_t**)(work + w.pd);
    KT_LAUNCH(k_moe1_up, dim3(kt_r8(F), k), dim3(64 * ((ksu + 1) / 2)), kt_moe1_up_lds(ksu), s, logits, E, k, rt,
                       wu, wd, F, H, (const float*)x, u, ids, gw, pd, ksu);
    KT_LAUNCH(k_moe1_down, dim3(kt_r8(H)), dim3(64 * ksd * ((k + 1) / 2)), kt_moe1_down_lds(k, ksd), s,
                       (const uint8_t* const*)pd, (const float*)gw, k, H, F, (const float*)u, yd, x, ysh, ksd);
    return 0;
  }
  /* 1: router, top-k, lists */
  KT_LAUNCH(k_moe_route, dim3(1), dim3(256), 0, s, logits, M, E, k, rt, ids, gw, cnt, off, xrow, where, act, nact,
                     (const float*)nullptr, 0, 0, (int8_t*)nullptr, 0, (float*)nullptr, 0);
  const int n = M * k;
  /* 2: up = W_e x[xrow[p]] per entry, x quantized in the staging */
  KtGroupedArgs a = {};
  a.wexp = (const uint8_t* const*)Wup;
  a.R = F; a.C = H; a.NU = H / 32;
  a.cnt = cnt; a.off = off; a.act = act; a.nact = nact; a.xrow = xrow;
  a.ldy = F; a.nrows = M; a.y = u;
  a.xf = x; a.ldxf = ldx;
  int rc = kt_grouped_xf<KT_FMT_Q8X>(a, E, n, M, s);
  if(rc) return rc;
  /* 3: down = W_e relu^2(u[p]) per entry, quantized in the staging */
  KtGroupedArgs b = {};
  b.wexp = (const uint8_t* const*)Wdown;
  b.R = H; b.C = F; b.NU = F / 32;
  b.cnt = cnt; b.off = off; b.act = act; b.nact = nact; b.xrow = nullptr;
  b.ldy = H; b.nrows = n; b.y = yd;
  b.xf = u; b.ldxf = F;
  rc = kt_grouped_xf<KT_FMT_Q8R>(b, E, n, M, s);
  if(rc) return rc;
  /* 4: x[t] += sum_j gw yd[where] (+ ysh) */
  KT_LAUNCH(k_moe_combine, dim3((H + 255) / 256, M), dim3(256), 0, s, (const float*)yd, ysh,
                     (const int*)where, (const float*)gw, k, H, x, ldx);
  return 0;
}

/* the workspace of kt_moe_decode_noalloc: one array per GPU, held until the process ends. In host code the array's
   name is not a device address; the address each device gives it is resolved once per device (kt_init, else the
   first call on the device) with hipGetSymbolAddress and only that address is used. Calls on one GPU share it:
   calls that overlap in time on one GPU race. */
#define KT_SCRATCH_BYTES ((size_t)4 << 20)
static __device__ __align__(256) uint8_t scratch[KT_SCRATCH_BYTES];
#define KT_MAX_DEVICES 64
static uint8_t* kt_scratch_ptr[KT_MAX_DEVICES];
static std::mutex kt_scratch_mu;
static int kt_scratch_resolve(int dev, uint8_t** out){
  if(dev < 0 || dev >= KT_MAX_DEVICES) return KT_INVALID;
  std::lock_guard<std::mutex> g(kt_scratch_mu);
  if(!kt_scratch_ptr[dev]){
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if(e != hipSuccess) return (int)e;
    if(!p) return KT_INVALID;
    kt_scratch_ptr[dev] = (uint8_t*)p;
  }
  *out = kt_scratch_ptr[dev];
  return 0;
}

template <int SRC>
static int kt_pack_launch(const uint8_t* bcodes, const uint16_t* dpm, int R, int C, void* W, void* stream){
  const int NG = C / 128;
  uint32_t* codes = (uint32_t*)W;
  uint16_t* scales = (uint16_t*)((uint8_t*)W + kt_code_bytes(R, NG));
  const long long nw = (long long)kt_code_bytes(R, NG) / 4;
  KT_LAUNCH((k_tern_pack<SRC>), dim3((unsigned)((nw + 255) / 256)), dim3(256), 0, kt_stream(stream),
                     bcodes, dpm, R, C, codes, scales);
  return 0;
}

/* launch records (kt_record_begin / kt_record_end): the calling thread's recording state */
static thread_local KtRecState kt_rec_tls;
static thread_local bool kt_rec_on = false;
KtRecState* kt_rec_state(){ return kt_rec_on ? &kt_rec_tls : nullptr; }

hipError_t kt_rec_push(const void* fn, dim3 g, dim3 b, size_t lds, int n, const void* const* vals,
                       const size_t* sizes, const size_t* aligns){
  KtRecState& r = kt_rec_tls;
  const int i = r.n++;
  if(r.err) return (hipError_t)r.err;
  if(i >= r.max) return hipSuccess;                              /* counted; kt_record_end reports the overflow */
  kt_launch& L = r.buf[i];
  memset(&L, 0, sizeof(L));
  hipFunction_t f = nullptr;
  hipError_t e = hipGetFuncBySymbol(&f, fn);
  if(e == hipSuccess && !f) e = hipErrorInvalidDeviceFunction;
  if(e == hipSuccess && (n > KT_REC_MAXARGS || lds > 0xFFFFFFFFu)) e = hipErrorInvalidValue;
  size_t o = 0;
  for(int a = 0; e == hipSuccess && a < n; ++a){
    o = (o + aligns[a] - 1) / aligns[a] * aligns[a];
    if(o + sizes[a] > sizeof(L.argbuf)){ e = hipErrorInvalidValue; break; }
    memcpy((uint8_t*)L.argbuf + o, vals[a], sizes[a]);
    L.off[a] = (unsigned)o;
    L.args[a] = (uint8_t*)L.argbuf + o;
    o += sizes[a];
  }
  if(e != hipSuccess){ r.err = (int)e; return e; }
  L.fn = (void*)f;
  L.grid[0] = g.x; L.grid[1] = g.y; L.grid[2] = g.z;
  L.block[0] = b.x; L.block[1] = b.y; L.block[2] = b.z;
  L.shmem = (unsigned)lds;
  L.nargs = n;
  return hipSuccess;
}

extern "C" {

int kt_version(void){ return KT_VERSION; }

int kt_init(int device){
  const hipError_t e = hipSetDevice(device);
  if(e != hipSuccess) return (int)e;
  uint8_t* p;
  return kt_scratch_resolve(device, &p);
}

const char* kt_error_string(int rc){ return hipGetErrorString((hipError_t)rc); }

int kt_replay(const kt_launch* recs, int n, void* const* streams, int nstreams){
  if(n < 0 || (n > 0 && !recs) || nstreams < 1 || nstreams > 16 || !streams) return KT_INVALID;
  for(int i = 0; i < n; ++i){
    const kt_launch& L = recs[i];
    const hipError_t e = hipModuleLaunchKernel((hipFunction_t)L.fn, L.grid[0], L.grid[1], L.grid[2], L.block[0],
                                               L.block[1], L.block[2], L.shmem, kt_stream(streams[i % nstreams]),
                                               (void**)L.args, nullptr);
    if(e != hipSuccess) return (int)e;
  }
  return 0;
}

int kt_record_begin(kt_launch* recs, int max){
  if(kt_rec_on || max < 0 || (max > 0 && !recs)) return KT_INVALID;
  kt_rec_tls.buf = recs; kt_rec_tls.max = max; kt_rec_tls.n = 0; kt_rec_tls.err = 0;
  kt_rec_on = true;
  return 0;
}

int kt_record_end(int* n){
  if(!kt_rec_on) return KT_INVALID;
  kt_rec_on = false;
  if(n) *n = kt_rec_tls.n;
  if(kt_rec_tls.err) return kt_rec_tls.err;
  return kt_rec_tls.n > kt_rec_tls.max ? KT_INVALID : 0;
}

/* ------------------------------------------------------------------ ternary weights */
size_t kt_tern_weight_bytes(int R, int C){
  if(R <= 0 || C <= 0 || C % 128) return 0;
  return kt_code_bytes(R, C / 128) + kt_scale_bytes(R, C / 128);
}

int kt_tern_pack(const uint8_t* bcodes, const uint16_t* dpm, int R, int C, void* W, void* stream){
  if(!bcodes || !dpm || !W || R <= 0 || C <= 0 || C % 128 || !kt_al(W, 16)) return KT_INVALID;
  return kt_pack_launch<0>(bcodes, dpm, R, C, W, stream);
}

int kt_tern_pack_layout(const uint8_t* wg4, const uint16_t* sg4, int R, int C, void* W, void* stream){
  if(!wg4 || !sg4 || !W || R <= 0 || C <= 0 || R % 16 || C % 512 || !kt_al(W, 16)) return KT_INVALID;
  return kt_pack_launch<1>(wg4, sg4, R, C, W, stream);
}

int kt_tern_pack_ptq1(const uint8_t* raw, int R, int C, int row0, int nrows, void* W, void* stream){
  if(nrows == 0) return 0;
  if(!raw || !W || R <= 0 || C <= 0 || C % 128 || !kt_al(W, 16) || row0 < 0 || row0 % KT_RG || nrows < 0
     || row0 + nrows > R || (row0 + nrows < R && nrows % KT_RG)) return KT_INVALID;
  const int NG = C / 128, nrg = (row0 + nrows == R ? kt_r8(R) : (row0 + nrows) / KT_RG) - row0 / KT_RG;
  uint32_t* codes = (uint32_t*)W;
  uint16_t* scales = (uint16_t*)((uint8_t*)W + kt_code_bytes(R, NG));
  const long long nw = (long long)nrg * NG * 64;
  KT_LAUNCH(k_tern_pack_ptq1, dim3((unsigned)((nw + 255) / 256)), dim3(256), 0, kt_stream(stream),
                     raw, R, C, row0, nrg, codes, scales);
  return 0;
}

int kt_quant_q8(const float* X, int ldx, int M, int C, int per_row, int8_t* XQ, int ldq, float* XS, int32_t* XA,
                void* stream){
  if(M == 0) return 0;
  if(!X || !XQ || !XS || !XA || M < 0 || C <= 0 || C % 128 || ldx < C || ldq < C || ldx % 2 || ldq % 16
     || !kt_al(X, 8) || !kt_al(XQ, 16) || per_row < 0 || per_row > 2) return KT_INVALID;
  KT_LAUNCH(k_quant_tern, dim3(M), dim3(256), 0, kt_stream(stream), X, ldx, C, per_row, XQ, ldq,
                     XS, (int*)XA);
  return 0;
}

/* ------------------------------------------------------------------ decode products */
int kt_decode_kslices(int C, int q8){
  if(C <= 0 || C % (q8 ? 32 : 128)) return 0;
  return kt_kslices(q8 ? C / 32 : C / 128);
}

int kt_tern_gemv(const void* W, int R, int C, const int8_t* XQ, int ldq, const float* XS, const int32_t* XA, int M,
                 float* Y, int ldy, int32_t* dbg, void* stream){
  const void* w[1] = {W};
  const int r[1] = {R}, l[1] = {ldy};
  float* y[1] = {Y};
  return kt_tern_gemv_n(1, w, r, y, l, C, XQ, ldq, XS, XA, M, dbg, stream);
}

int kt_tern_gemv3(const void* W0, int R0, float* Y0, const void* W1, int R1, float* Y1, const void* W2, int R2,
                  float* Y2, int C, const int8_t* XQ, int ldq, const float* XS, const int32_t* XA, int M,
                  void* stream){
  const void* w[3] = {W0, W1, W2};
  const int r[3] = {R0, R1, R2};
  float* y[3] = {Y0, Y1, Y2};
  const int n = R1 <= 0 ? 1 : R2 <= 0 ? 2 : 3;
  return kt_tern_gemv_n(n, w, r, y, r, C, XQ, ldq, XS, XA, M, NULL, stream);
}

int kt_tern_sum(const float* P, float* y, int R, int M, int sp, void* stream){
  if(M == 0) return 0;
  if(!P || !y || R <= 0 || M < 0 || M > 65535 || sp <= 0) return KT_INVALID;
  KT_LAUNCH(k_tern_sum, dim3((unsigned)((R + 255) / 256), (unsigned)M), dim3(256), 0, kt_stream(stream), P, y,
                     R, M, sp);
  return 0;
}


/* ------------------------------------------------------------------ prefill product */
/* per_row = 0: the reference's per-group expression on 128 x 128 blocks. per_row = 1: the per-row order, on small
   blocks (128 tokens x 64 rows) while a grid of 128 x 128 blocks would have fewer than KT_RS_BLOCKS blocks (4 a CU),
   else on 128 x 128 blocks; both run the same per-element chain, so the bits do not depend on the choice (measured
   on MI355X, config 2: gate/up [12288 x 4096] at 512 tokens 60.0 -> 56.5 us on the small blocks, at 2048 tokens
   190.8 against 202.6 us on the large ones) */
int kt_tern_gemm(const void* W, int R, int C, const int8_t* XQ, int ldq, const float* XS, const int32_t* XA,
                 int per_row, int M, float* Y, uint16_t* Y16, int ldy, int32_t* dbg, void* stream){
  (void)XA;                                                  /* signed trits on the matrix cores: no digit offset */
  if(M == 0) return 0;
  if(!W || !XQ || !XS || (!Y && !Y16) || R <= 0 || M < 0 || C <= 0 || C % 128 || ldq < C || ldq % 16 || ldy < R
     || !kt_al(W, 16) || !kt_al(XQ, 16) || (per_row != 0 && per_row != 1)) return KT_INVALID;
  const int NG = C / 128;
  const uint32_t* codes = (const uint32_t*)W;
  const uint16_t* scales = (const uint16_t*)((const uint8_t*)W + kt_code_bytes(R, NG));
  /* both kernels read through buffer resources with 32-bit offsets */
  if((long long)M * ldq >= (1ll << 31) || (long long)M * NG * 4 >= (1ll << 31) || kt_code_bytes(R, NG) >= (1ull << 31))
    return KT_INVALID;
  hipStream_t s = kt_stream(stream);
  if(per_row && (long long)((R + 127) / 128) * ((M + 127) / 128) < KT_RS_BLOCKS){
    /* one 32 x 32 tile a wave, 8 waves: 128 tokens x 64 rows */
    const dim3 grid((R + 63) / 64, (M + 127) / 128);
    if(dbg) KT_LAUNCH((k_tern_gemm_rs1<4, 2, 3, true>), grid, dim3(512), 0, s, codes, scales, R, NG, XQ, ldq,
                               XS, M, Y, Y16, ldy, dbg);
    else KT_LAUNCH((k_tern_gemm_rs1<4, 2, 3, false>), grid, dim3(512), 0, s, codes, scales, R, NG, XQ, ldq,
                            XS, M, Y, Y16, ldy, dbg);
    return 0;
  }
  const dim3 grid((R + 127) / 128, (M + 127) / 128);
#define KT_TG(DBG, RS) KT_LAUNCH((k_tern_gemm<DBG, RS>), grid, dim3(256), 0, s, codes, scales, R, NG, XQ, ldq, \
                                          XS, M, Y, Y16, ldy, dbg)
  if(per_row){ if(dbg) KT_TG(true, true); else KT_TG(false, true); }
  else { if(dbg) KT_TG(true, false); else KT_TG(false, false); }
#undef KT_TG
  return 0;
}

/* the current device's CU count, queried once per device */
static int kt_cu_count(int* cus){
  static int cache[64];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if(e != hipSuccess) return (int)e;
  if(dev < 0 || dev >= 64) return KT_INVALID;
  if(!cache[dev]){
    int n = 0;
    e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if(e != hipSuccess) return (int)e;
    cache[dev] = n;
  }
  *cus = cache[dev];
  return 0;
}

size_t kt_tern_expand_bytes(int R, int C){
  if(R <= 0 || C <= 0 || C % 128) return 0;
  return (size_t)kt_r8(R) * KT_RG * C;
}

int kt_tern_expand(const void* W, int R, int C, int8_t* W8, void* stream){
  if(!W || !W8 || R <= 0 || C <= 0 || C % 128 || !kt_al(W, 16) || !kt_al(W8, 16)) return KT_INVALID;
  const int NU = C / 128;
  const long long nq = (long long)kt_r8(R) * NU * 16;                     /* kt2 chunks */
  KT_LAUNCH(k_tern_expand, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, kt_stream(stream), (const uint4*)W, NU,
            nq, C, W8);
  return 0;
}

int kt_tern_gemm8(const int8_t* W8, const void* W, int R, int C, const int8_t* XQ, int ldq, const float* XS, int M,
                  float* Y, uint16_t* Y16, int ldy, int32_t* dbg, void* stream){
  if(M == 0) return 0;
  if(!W8 || !W || !XQ || !XS || (!Y && !Y16) || R <= 0 || M < 0 || C <= 0 || C % 128 || ldq < C || ldq % 16
     || ldy < R || !kt_al(W, 16) || !kt_al(W8, 16) || !kt_al(XQ, 16)) return KT_INVALID;
  const int NG = C / 128;
  /* 32-bit buffer offsets, an out-of-range offset at 2^31 */
  if((long long)M * ldq >= (1ll << 31) || (long long)kt_r8(R) * KT_RG * C >= (1ll << 31)) return KT_INVALID;
  const uint16_t* scales = (const uint16_t*)((const uint8_t*)W + kt_code_bytes(R, NG));
  /* a grid short of 0.7 of a 128 x 256 tile a CU, or outputs the kernel's 16-byte row stores cannot take, run the
     packed-trit product instead (the same per-row numbers and order, so the same bits) */
  int cus = 0;
  const int ec = kt_cu_count(&cus);
  if(ec) return ec;
  const bool aligned = ldy % 8 == 0 && (!Y || kt_al(Y, 16)) && (!Y16 || kt_al(Y16, 16));   /* 16-byte output rows */
#ifndef KT_G8_MIN_PCT
#define KT_G8_MIN_PCT 70              /* tiles a CU, percent (measured on MI355X: gate/up [12288 x 4096] at 512 tokens,
                                         192 tiles on 256 CUs, 53.7 -> 41.9 us over the packed-trit kernel) */
#endif
  if((long long)((kt_r8(R) * KT_RG + 255) / 256) * ((M + 127) / 128) * 100 < (long long)cus * KT_G8_MIN_PCT || !aligned)
    return kt_tern_gemm(W, R, C, XQ, ldq, XS, nullptr, 1, M, Y, Y16, ldy, dbg, stream);
  const size_t lds = kt_gemm8_lds();
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, []{
    const size_t n = kt_gemm8_lds();
    attr = hipFuncSetAttribute((const void*)k_tern_gemm8<false>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)n);
    if(attr == hipSuccess)
      attr = hipFuncSetAttribute((const void*)k_tern_gemm8<true>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)n);
  });
  if(attr != hipSuccess) return (int)attr;
  /* one block a CU (its LDS), each taking tiles blockIdx.x, + grid, ... */
  const int gx = (kt_r8(R) * KT_RG + 255) / 256, gy = (M + 127) / 128;
  const dim3 grid(gx * gy < cus ? gx * gy : cus);
  if(dbg) KT_LAUNCH(k_tern_gemm8<true>, grid, dim3(512), lds, kt_stream(stream), W8, scales, R, C, XQ, ldq, XS, M, Y,
                    Y16, ldy, dbg, gx, gy);
  else KT_LAUNCH(k_tern_gemm8<false>, grid, dim3(512), lds, kt_stream(stream), W8, scales, R, C, XQ, ldq, XS, M, Y,
                 Y16, ldy, dbg, gx, gy);
  return 0;
}

/* ------------------------------------------------------------------ q8_0 */
size_t kt_q8_weight_bytes(int R, int C){
  if(R <= 0 || C <= 0 || C % 32) return 0;
  return kt_code_bytes(R, C / 32) + kt_scale_bytes(R, C / 32);
}

int kt_q8_pack(const uint8_t* rows, int R, int C, void* W, void* stream){
  if(!rows || !W || R <= 0 || C <= 0 || C % 32 || !kt_al(W, 16)) return KT_INVALID;
  const int NB = C / 32;
  uint32_t* codes = (uint32_t*)W;
  uint16_t* scales = (uint16_t*)((uint8_t*)W + kt_code_bytes(R, NB));
  const long long nw = (long long)kt_code_bytes(R, NB) / 4;
  KT_LAUNCH(k_q8_pack, dim3((unsigned)((nw + 255) / 256)), dim3(256), 0, kt_stream(stream), rows, R, C,
                     codes, scales);
  return 0;
}

int kt_q8_quant(const float* X, int ldx, int M, int C, int act, int8_t* Q, int ldq, float* D, int ldd, void* stream){
  if(M == 0) return 0;
  if(!X || !Q || !D || M < 0 || C <= 0 || C % 32 || ldx < C || ldq < C || ldd < C / 32 || !kt_al(X, 16) || ldx % 4
     || !kt_al(Q, 4) || ldq % 4) return KT_INVALID;
  const int NB = C / 32;
  KT_LAUNCH(k_quant_q8, dim3((NB + 31) / 32, M), dim3(256), 0, kt_stream(stream), X, ldx, C, act ? 1 : 0, Q,
                     ldq, D, ldd);
  return 0;
}

int kt_q8_gemv(const void* W, int R, int C, const int8_t* Q, int ldq, const float* D, int ldd, int M, float* Y,
               int ldy, int32_t* dbg, void* stream){
  if(M == 0) return 0;
  if(!W || !Q || !D || !Y || R <= 0 || M < 0 || C <= 0 || C % 32 || ldq < C || ldq % 16 || ldd < C / 32 || ldy < R
     || !kt_al(W, 16) || !kt_al(Q, 16)) return KT_INVALID;
  const int NB = C / 32;
  KtGemvArgs a = {};
  a.mat[0].codes = (const uint32_t*)W;
  a.mat[0].scales = (const uint16_t*)((const uint8_t*)W + kt_code_bytes(R, NB));
  a.mat[0].y = Y; a.mat[0].R = R; a.mat[0].ldy = ldy; a.mat[0].rg0 = 0;
  a.nmat = 1; a.NU = NB;
  a.ldq = ldq; a.ldxs = ldd;
  a.M = M;
  const int ks = kt_kslices(NB);
  if(M >= KT_Q8_MMA_MIN && ks <= KT_Q8_MMA_KS && (long long)M * ldq < (1ll << 31)){
    /* the matrix-core product (the same numbers and tree): tiles of 32 rows, all tokens a block */
    const dim3 grid((kt_r8(R) + 3) / 4), block(64 * ks);
    const size_t lds = (size_t)ks * 16 * 32 * 4 + (size_t)ks * 256 * 4;          /* slice sums, D */
    const KtGroupedArgs ga = {};
    if(dbg) KT_LAUNCH((k_q8_mma<false, true, false>), grid, block, lds, kt_stream(stream), a, ga, Q, D, dbg, ks);
    else KT_LAUNCH((k_q8_mma<false, false, false>), grid, block, lds, kt_stream(stream), a, ga, Q, D, dbg, ks);
    return 0;
  }
  return kt_launch_gemv<KT_FMT_Q8>(a, kt_r8(R), Q, D, NULL, dbg, kt_stream(stream));
}

/* ------------------------------------------------------------------ MoE */
/* the router of kt_moe_*_r: the scoring and its operands (include/kt.h KT_SCORE_*) */
static bool kt_router(int score, const float* bias, float scale, KtRouter& rt){
  rt.score = score; rt.bias = bias; rt.scale = scale;
  if(score == KT_SCORE_SOFTMAX) return true;
  return score == KT_SCORE_SIGMOID && bias != nullptr;
}

int kt_moe_topk_r(const float* logits, int M, int E, int k, int score, const float* bias, float scale, int* ids,
                  float* gw, void* stream){
  KtRouter rt;
  if(!kt_router(score, bias, scale, rt)) return KT_INVALID;
  if(M == 0) return 0;
  if(!logits || !ids || !gw || M < 0 || E <= 0 || E > 1024 || k <= 0 || k > 16 || k > E) return KT_INVALID;
  KT_LAUNCH(k_moe_topk, dim3(M), dim3(64), 0, kt_stream(stream), logits, E, k, rt, ids, gw);
  return 0;
}

int kt_moe_topk(const float* logits, int M, int E, int k, int* ids, float* gw, void* stream){
  return kt_moe_topk_r(logits, M, E, k, KT_SCORE_SOFTMAX, nullptr, 1.0f, ids, gw, stream);
}

int kt_moe_route_r(const float* logits, int M, int E, int k, int score, const float* bias, float scale, int* ids,
                   float* gw, int* cnt, int* off, int* xrow, int* where, int* act, int* nact, const float* x, int ldx,
                   int H, int8_t* Q, int ldq, float* D, int ldd, void* stream){
  KtRouter rt;
  if(!kt_router(score, bias, scale, rt)) return KT_INVALID;
  if(!logits || !ids || !gw || !cnt || !off || !xrow || !where || !act || !nact || M < 0 || E <= 0 || E > 1024 ||
     k <= 0 || k > 16 || k > E || M > 64 || (long long)M * k > 64) return KT_INVALID;
  if(x && (H <= 0 || H % 32 || ldx < H || !Q || ldq < H || !D || ldd < H / 32)) return KT_INVALID;
  KT_LAUNCH(k_moe_route, dim3(1), dim3(256), 0, kt_stream(stream), logits, M, E, k, rt, ids, gw, cnt, off, xrow,
            where, act, nact, x, ldx, H, Q, ldq, D, ldd);
  return 0;
}

int kt_moe_route(const float* logits, int M, int E, int k, int* ids, float* gw, int* cnt, int* off, int* xrow,
                 int* where, int* act, int* nact, const float* x, int ldx, int H, int8_t* Q, int ldq, float* D, int ldd,
                 void* stream){
  return kt_moe_route_r(logits, M, E, k, KT_SCORE_SOFTMAX, nullptr, 1.0f, ids, gw, cnt, off, xrow, where, act, nact,
                        x, ldx, H, Q, ldq, D, ldd, stream);
}

int kt_moe_sort(const int* ids, int M, int k, int E, int* cnt, int* off, int* xrow, int* where, int* act, int* nact,
                void* stream){
  if(!ids || !cnt || !off || !xrow || !where || !act || !nact || M < 0 || k <= 0 || k > 16 || E <= 0 || E > 1024
     || (long long)M * k > (1ll << 30)) return KT_INVALID;
  KT_LAUNCH(k_moe_sort, dim3(1), dim3(1024), (size_t)16 * E * 4, kt_stream(stream), ids, M * k, E, cnt, off,
                     xrow, where, act, nact, k);
  return 0;
}

int kt_q8_grouped(const void* const* Wexp, int R, int C, int E, const int* cnt, const int* off, const int* act,
                  const int* nact, const int* xrow, int nentries, int M, const int8_t* Q, int ldq, const float* D,
                  int ldd, float* Y, int ldy, int32_t* dbg, void* stream){
  if(nentries == 0) return 0;
  if(!Wexp || !cnt || !off || !act || !nact || !Q || !D || !Y || R <= 0 || C <= 0 || C % 32 || E <= 0
     || nentries < 0 || M <= 0 || ldq < C || ldq % 16 || ldd < C / 32 || ldy < R || !kt_al(Q, 16))
    return KT_INVALID;
  KtGroupedArgs a = {};
  a.wexp = (const uint8_t* const*)Wexp;
  a.R = R; a.C = C; a.NU = C / 32;
  a.cnt = cnt; a.off = off; a.act = act; a.nact = nact; a.xrow = xrow;
  a.ldq = ldq; a.ldd = ldd; a.ldy = ldy; a.nrows = xrow ? M : nentries;
  a.y = Y;
  const int ks = kt_kslices(a.NU);
  const int ny = E < nentries ? E : nentries;
  hipStream_t s = kt_stream(stream);
  /* the matrix-core kernel reads the input rows through a buffer resource with 32-bit offsets */
  if(nentries >= 4 * ny && ks <= KT_Q8_MMA_KS && (long long)a.nrows * ldq < (1ll << 31)){
    /* 4 or more entries an active expert on average: the matrix-core product per (32-row tile, active expert), the
       expert's whole list in passes of 16 (the same numbers and tree) */
    const dim3 grid((kt_r8(R) + 3) / 4, ny), block(64 * ks);
    const size_t lds = (size_t)ks * 16 * 32 * 4 + (size_t)ks * 256 * 4;          /* slice sums, D */
    const KtGemvArgs da = {};
    if(ks > 2){
      /* two waves a block taking the slices in turn (the same slice sums in the same order): blocks of 2 waves at
         2 waves a SIMD fill every wave slot of a CU, where KS-wave blocks left slots empty (6 slices: 6 of 8) and
         with them weight bytes in flight (measured on MI355X, config 4 M=256: up 223 -> 162 us, down 161 -> 158 us;
         one wave a block 169 / 157, three 185 / 210) */
      const dim3 blk(128);
      if(dbg) KT_LAUNCH((k_q8_mma<true, true, true>), grid, blk, lds, s, da, a, Q, D, dbg, ks);
      else KT_LAUNCH((k_q8_mma<true, false, true>), grid, blk, lds, s, da, a, Q, D, dbg, ks);
    } else if(dbg) KT_LAUNCH((k_q8_mma<true, true, false>), grid, block, lds, s, da, a, Q, D, dbg, ks);
    else KT_LAUNCH((k_q8_mma<true, false, false>), grid, block, lds, s, da, a, Q, D, dbg, ks);
    return 0;
  }
  /* the decode product per (row group, active expert), the expert's list in chunks of up to 4 tokens */
#ifndef KT_GRP_MT
#define KT_GRP_MT 2                   /* tokens a chunk in the grouped product (registers: more waves resident) */
#endif
  int mt = M <= 1 ? 1 : M <= 2 ? 2 : 4;
  if(mt > KT_GRP_MT) mt = KT_GRP_MT;
  while(mt > 1 && (mt == 4 ? KtFlat<KT_FMT_Q8, 4>::lds(ks) : KtFlat<KT_FMT_Q8, 2>::lds(ks)) > 65536) mt >>= 1;
  const dim3 grid(kt_r8(R), ny), block(64 * ks);
  const KtGemvArgs da = {};
#define KT_GL(K, MT) do { const size_t lds = KtFlat<KT_FMT_Q8, MT>::lds(ks); \
    if(dbg) KT_LAUNCH((K<KT_FMT_Q8, MT, true, true>), grid, block, lds, s, da, a, Q, D, nullptr, dbg, ks); \
    else KT_LAUNCH((K<KT_FMT_Q8, MT, false, true>), grid, block, lds, s, da, a, Q, D, nullptr, dbg, ks); } while(0)
  if(mt == 4) KT_GL(k_gemv_flat, 4); else if(mt == 2) KT_GL(k_gemv_flat, 2); else KT_GL(k_gemv_flat1, 1);
#undef KT_GL
  return 0;
}

int kt_moe_combine(const float* yd, const float* ysh, const int* where, const float* gw, int M, int k, int cols,
                   float* x, void* stream){
  if(M == 0) return 0;
  if(!yd || !where || !gw || !x || M < 0 || M > 65535 || k <= 0 || k > 16 || cols <= 0) return KT_INVALID;
  KT_LAUNCH(k_moe_combine, dim3((cols + 255) / 256, M), dim3(256), 0, kt_stream(stream), yd, ysh, where, gw,
                     k, cols, x, cols);
  return 0;
}

size_t kt_moe_decode_workspace(int M, int k, int E, int H, int F){
  KtMoeWork w;
  return kt_moe_work(M, k, E, H, F, w) ? w.total : 0;
}

int kt_moe_decode_r(const void* const* Wup, const void* const* Wdown, int E, int H, int F, int k, int score,
                    const float* bias, float scale, const float* logits, int M, float* x, int ldx, const float* ysh,
                    void* work, size_t work_bytes, void* stream){
  KtRouter rt;
  if(!kt_router(score, bias, scale, rt)) return KT_INVALID;
  if(M == 0) return 0;
  return kt_moe_decode_run(Wup, Wdown, E, H, F, k, rt, logits, M, x, ldx, ysh, (uint8_t*)work, work_bytes,
                           kt_stream(stream));
}

int kt_moe_decode(const void* const* Wup, const void* const* Wdown, int E, int H, int F, int k, const float* logits,
                  int M, float* x, int ldx, const float* ysh, void* work, size_t work_bytes, void* stream){
  return kt_moe_decode_r(Wup, Wdown, E, H, F, k, KT_SCORE_SOFTMAX, nullptr, 1.0f, logits, M, x, ldx, ysh, work,
                         work_bytes, stream);
}

size_t kt_moe_decode_noalloc_max(void){ return KT_SCRATCH_BYTES; }

int kt_moe_decode_noalloc(const void* const* Wup, const void* const* Wdown, int E, int H, int F, int k,
                          const float* logits, int M, float* x, int ldx, const float* ysh, void* stream){
  if(M == 0) return 0;
  KtMoeWork w;
  if(!kt_moe_work(M, k, E, H, F, w)) return KT_INVALID;
  if(w.total > KT_SCRATCH_BYTES) return KT_INVALID;               /* beyond the static workspace */
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if(e != hipSuccess) return (int)e;
  uint8_t* p = nullptr;
  const int rc = kt_scratch_resolve(dev, &p);
  if(rc) return rc;
  const KtRouter rt = {KT_SCORE_SOFTMAX, 1.0f, nullptr};
  return kt_moe_decode_run(Wup, Wdown, E, H, F, k, rt, logits, M, x, ldx, ysh, p, KT_SCRATCH_BYTES,
                           kt_stream(stream));
}

/* ------------------------------------------------------------------ fused input producers (kt_fold.hip) */
static bool kt_fold_shape(int M, int C, int HB, const float* sg, int8_t* XQ, int ldq, float* XS, int32_t* XA){
  return M >= 0 && M <= 65535 && C >= 512 && C <= (1 << 20) && (HB == 512 || HB == 1024 || HB == 4096)
      && C % HB == 0 && sg && XQ && XS && XA && ldq >= C;
}

static int kt_fold_run(int mode, const KtFoldArgs& a, int M, void* stream){
  if(M == 0) return 0;
  return (int)kt_fold_launch(mode, a, M, kt_stream(stream));
}

int kt_rmsfold_q8(const float* x, int ldx, const float* r, int ldr, int nparts, const float* w, const float* sg, int M,
                  int C, int HB, float* xw, int ldxw, float* xn, int ldxn, float* xo, int ldxo, int8_t* XQ, int ldq,
                  float* XS, int32_t* XA, void* stream){
  const int hp = (HB & KT_HP) ? 1 : 0;                      /* HB | KT_HP: two int8 rows a token */
  HB &= ~KT_HP;
  if(!kt_fold_shape(M, C, HB, sg, XQ, ldq, XS, XA) || C > 8192 || !x || !w || ldx < C || nparts < 0 || nparts > 8
     || (nparts > 0 && (!r || ldr < nparts * C)) || (xw && ldxw < C) || (xn && ldxn < C) || (xo && ldxo < C))
    return KT_INVALID;
  KtFoldArgs a = {x, ldx, r, ldr, nparts, w, sg, 1, 1, 1, xw, ldxw, xn, ldxn, xo, ldxo, C, HB, XQ, ldq, XS, XA, hp};
  return kt_fold_run(0, a, M, stream);
}

int kt_fold_q8(const float* x, int ldx, const float* sg, int M, int C, int HB, float* xo, int ldxo, int8_t* XQ,
               int ldq, float* XS, int32_t* XA, void* stream){
  const int hp = (HB & KT_HP) ? 1 : 0;                      /* HB | KT_HP: two int8 rows a token */
  HB &= ~KT_HP;
  if(!kt_fold_shape(M, C, HB, sg, XQ, ldq, XS, XA) || !x || ldx < C || (xo && ldxo < C)) return KT_INVALID;
  KtFoldArgs a = {x, ldx, nullptr, 0, 0, nullptr, sg, 1, 1, 1, nullptr, 0, nullptr, 0, xo, ldxo, C, HB, XQ, ldq, XS, XA, hp};
  return kt_fold_run(1, a, M, stream);
}

int kt_smfold_q8(const float* a_, int lda, const float* b, int ldb, const float* sg, int hd, int nk, int rep, int M,
                 int C, int HB, float* xo, int ldxo, int8_t* XQ, int ldq, float* XS, int32_t* XA, void* stream){
  const int hp = (HB & KT_HP) ? 1 : 0;                      /* HB | KT_HP: two int8 rows a token */
  HB &= ~KT_HP;
  if(!kt_fold_shape(M, C, HB, sg, XQ, ldq, XS, XA) || !a_ || !b || lda < C || ldb < C || (xo && ldxo < C) || rep < 1
     || (rep > 1 && (hd <= 0 || nk <= 0 || (long long)hd * nk * rep != C)))
    return KT_INVALID;
  KtFoldArgs a = {a_, lda, b, ldb, 0, nullptr, sg, hd, nk, rep, nullptr, 0, nullptr, 0, xo, ldxo, C, HB, XQ, ldq, XS,
                  XA, hp};
  return kt_fold_run(2, a, M, stream);
}

}  /* extern "C" */
