/* kt_api.hip - the C ABI of libkt_gfx950.so: host-side validation, launch plans and launches. Every entry point
   takes caller-owned device pointers and a stream (NULL = the null stream), never allocates, never synchronizes,
   and returns a hipError_t as int (0 = success; hipErrorInvalidValue for shapes or strides the kernels do not
   take). The declarations and the reference interfaces they replace are in include/kt.h. */
#include "kt_common.h"
#include "../../include/kt.h"

template <int FMT, int MT> __global__ void k_gemv(const KtGemvArgs, const int8_t*, const float*, const int*, int32_t*);
template <int MT> __global__ void k_q8_grouped(const KtGroupedArgs);
extern "C" __global__ void k_tern_pack(const uint8_t*, const uint16_t*, int, int, int, uint32_t*, uint16_t*);
extern "C" __global__ void k_q8_pack(const uint8_t*, int, int, int, uint32_t*, uint16_t*);
extern "C" __global__ void k_quant_tern(const float*, int, int, int, int8_t*, int, float*, int*);
extern "C" __global__ void k_quant_q8(const float*, int, int, int, int8_t*, int, float*, int);
extern "C" __global__ void k_tern_sum(const float*, float*, int, int, int);
extern "C" __global__ void k_tern_gemm(const uint32_t*, const uint16_t*, int, int, int, const int8_t*, int,
                                       const float*, int, float*, uint16_t*, int, int32_t*);
extern "C" __global__ void k_moe_topk(const float*, int, int, int*, float*);
extern "C" __global__ void k_moe_sort(const int*, int, int, int*, int*, int*, int*, int*, int*, int);
extern "C" __global__ void k_moe_combine(const float*, const float*, const int*, const float*, int, int, float*);

#define KT_INVALID ((int)hipErrorInvalidValue)
#define KT_LAUNCH_CHECK() do { const hipError_t _e = hipGetLastError(); if(_e != hipSuccess) return (int)_e; } while(0)

static inline hipStream_t kt_stream(void* s){ return (hipStream_t)s; }
static inline int kt_rp(int R){ return (R + KT_TR - 1) / KT_TR * KT_TR; }
static inline bool kt_al(const void* p, size_t a){ return ((uintptr_t)p % a) == 0; }

/* the K split of a launch over ntiles 64-row tiles and NU units: a function of the shape only (never of M), so a
   token's result does not depend on how many tokens share the pass, and is fixed across runs */
static int kt_nsplit(int ntiles, int NU, int min_units){
  const int target_blocks = KT_TARGET_WAVES / KT_WAVES;
  int sp = (target_blocks + ntiles - 1) / ntiles;
  const int cap = NU / (KT_WAVES * min_units);
  if(sp > cap) sp = cap;
  if(sp < 1) sp = 1;
  return sp;
}

/* workspace: the arrival counters of every launch live in a fixed prefix (zero between launches, whatever shape
   used the workspace before), the partial sums after it */
#define KT_WS_COUNTERS 16384
#define KT_WS_PARTS ((size_t)KT_WS_COUNTERS * 4)
static size_t kt_ws_bytes(int nsplit, int M, int ntiles){
  return nsplit <= 1 ? 0 : KT_WS_PARTS + (size_t)nsplit * M * ntiles * KT_TR * 4;
}
static int kt_ws_set(KtGemvArgs& a, void* ws){
  if(a.nsplit <= 1) return 0;
  const int mt = a.M <= 1 ? 1 : a.M <= 2 ? 2 : a.M <= 4 ? 4 : a.M <= 8 ? 8 : 16;
  if(!ws || !kt_al(ws, 16) || (long long)((a.M + mt - 1) / mt) * a.ntiles > KT_WS_COUNTERS) return KT_INVALID;
  a.counters = (int*)ws;
  a.parts = (float*)((uint8_t*)ws + KT_WS_PARTS);
  return 0;
}

static int kt_mt(int M){ return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16; }

template <int FMT>
static int kt_launch_gemv(KtGemvArgs& a, int ntiles, hipStream_t s){
  const int mt = kt_mt(a.M), npass = (a.M + mt - 1) / mt;
  const dim3 grid(ntiles, a.nsplit, npass), block(256);
  switch(mt){
    case 1: hipLaunchKernelGGL((k_gemv<FMT, 1>), grid, block, 0, s, a, a.xq, a.xs, a.xa, a.dbg); break;
    case 2: hipLaunchKernelGGL((k_gemv<FMT, 2>), grid, block, 0, s, a, a.xq, a.xs, a.xa, a.dbg); break;
    case 4: hipLaunchKernelGGL((k_gemv<FMT, 4>), grid, block, 0, s, a, a.xq, a.xs, a.xa, a.dbg); break;
    case 8: hipLaunchKernelGGL((k_gemv<FMT, 8>), grid, block, 0, s, a, a.xq, a.xs, a.xa, a.dbg); break;
    default: hipLaunchKernelGGL((k_gemv<FMT, 16>), grid, block, 0, s, a, a.xq, a.xs, a.xa, a.dbg); break;
  }
  KT_LAUNCH_CHECK();
  return 0;
}

extern "C" {

int kt_version(void){ return KT_VERSION; }

int kt_init(int device){ return (int)hipSetDevice(device); }

const char* kt_error_string(int rc){ return hipGetErrorString((hipError_t)rc); }

/* ------------------------------------------------------------------ ternary weights */
size_t kt_tern_weight_bytes(int R, int C){
  if(R <= 0 || C <= 0 || C % 128) return 0;
  const size_t Rp = (size_t)kt_rp(R), NG = (size_t)(C / 128);
  return Rp * NG * 32 + Rp * NG * 2;
}

int kt_tern_pack(const uint8_t* bcodes, const uint16_t* dpm, int R, int C, void* W, void* stream){
  if(!bcodes || !dpm || !W || R <= 0 || C <= 0 || C % 128 || !kt_al(W, 16)) return KT_INVALID;
  const int Rp = kt_rp(R), NG = C / 128;
  uint32_t* codes = (uint32_t*)W;
  uint16_t* scales = (uint16_t*)((uint8_t*)W + (size_t)Rp * NG * 32);
  const long long nw = (long long)Rp * NG * 8;
  hipLaunchKernelGGL(k_tern_pack, dim3((unsigned)((nw + 255) / 256)), dim3(256), 0, kt_stream(stream),
                     bcodes, dpm, R, C, Rp, codes, scales);
  KT_LAUNCH_CHECK();
  return 0;
}

int kt_quant_q8(const float* X, int ldx, int M, int C, int per_row, int8_t* XQ, int ldq, float* XS, int32_t* XA,
                void* stream){
  if(M == 0) return 0;
  if(!X || !XQ || !XS || !XA || M < 0 || C <= 0 || C % 128 || ldx < C || ldq < C || ldx % 2 || ldq % 16
     || !kt_al(X, 8) || !kt_al(XQ, 16)) return KT_INVALID;
  hipLaunchKernelGGL(k_quant_tern, dim3(M), dim3(256), 0, kt_stream(stream), X, ldx, C, per_row ? 1 : 0, XQ, ldq,
                     XS, (int*)XA);
  KT_LAUNCH_CHECK();
  return 0;
}

/* ------------------------------------------------------------------ decode products */
int kt_tern_gemv_splits(int R, int C){
  if(R <= 0 || C <= 0 || C % 128) return 0;
  return kt_nsplit(kt_rp(R) / KT_TR, C / 128, KT_MIN_UNITS);
}

size_t kt_tern_gemv_workspace(int R, int C, int M){
  if(R <= 0 || C <= 0 || C % 128 || M <= 0) return 0;
  const int ntiles = kt_rp(R) / KT_TR, sp = kt_nsplit(ntiles, C / 128, KT_MIN_UNITS), mt = kt_mt(M);
  (void)mt;
  return kt_ws_bytes(sp, M, ntiles);
}

static int kt_tern_gemv_n(int nmat, const void* const* W, const int* Rs, float* const* Ys, const int* ldys, int C,
                          const int8_t* XQ, int ldq, const float* XS, const int32_t* XA, int M, int32_t* dbg,
                          void* ws, void* stream){
  if(M == 0) return 0;
  if(M < 0 || C <= 0 || C % 128 || !XQ || !XS || !XA || ldq < C || ldq % 16 || !kt_al(XQ, 16)) return KT_INVALID;
  KtGemvArgs a = {};
  const int NG = C / 128;
  int tiles = 0;
  for(int i = 0; i < nmat; ++i){
    if(!W[i] || !Ys[i] || Rs[i] <= 0 || ldys[i] < Rs[i] || !kt_al(W[i], 16)) return KT_INVALID;
    const int Rp = kt_rp(Rs[i]);
    a.mat[i].codes = (const uint32_t*)W[i];
    a.mat[i].scales = (const uint16_t*)((const uint8_t*)W[i] + (size_t)Rp * NG * 32);
    a.mat[i].y = Ys[i];
    a.mat[i].R = Rs[i];
    a.mat[i].ldy = ldys[i];
    a.mat[i].tile0 = tiles;
    tiles += Rp / KT_TR;
  }
  if(dbg && nmat != 1) return KT_INVALID;
  a.nmat = nmat;
  a.NU = NG;
  a.xq = XQ; a.ldq = ldq; a.xs = XS; a.xa = (const int*)XA; a.ldxs = NG;
  a.M = M;
  a.dbg = dbg;
  a.nsplit = kt_nsplit(tiles, NG, KT_MIN_UNITS);
  a.Rtot = tiles * KT_TR;
  a.ntiles = tiles;
  if(kt_ws_set(a, ws)) return KT_INVALID;
  return kt_launch_gemv<KT_FMT_TERN>(a, tiles, kt_stream(stream));
}

int kt_tern_gemv(const void* W, int R, int C, const int8_t* XQ, int ldq, const float* XS, const int32_t* XA, int M,
                 float* Y, int ldy, int32_t* dbg, void* ws, void* stream){
  const void* w[1] = {W};
  const int r[1] = {R}, l[1] = {ldy};
  float* y[1] = {Y};
  return kt_tern_gemv_n(1, w, r, y, l, C, XQ, ldq, XS, XA, M, dbg, ws, stream);
}

size_t kt_tern_gemv3_workspace(int R0, int R1, int R2, int C, int M){
  if(C <= 0 || C % 128 || M <= 0 || R0 <= 0) return 0;
  const int tiles = kt_rp(R0) / KT_TR + (R1 > 0 ? kt_rp(R1) / KT_TR : 0) + (R2 > 0 ? kt_rp(R2) / KT_TR : 0);
  return kt_ws_bytes(kt_nsplit(tiles, C / 128, KT_MIN_UNITS), M, tiles);
}

int kt_tern_gemv3(const void* W0, int R0, float* Y0, const void* W1, int R1, float* Y1, const void* W2, int R2,
                  float* Y2, int C, const int8_t* XQ, int ldq, const float* XS, const int32_t* XA, int M, void* ws,
                  void* stream){
  const void* w[3] = {W0, W1, W2};
  const int r[3] = {R0, R1, R2};
  float* y[3] = {Y0, Y1, Y2};
  const int n = R1 <= 0 ? 1 : R2 <= 0 ? 2 : 3;
  return kt_tern_gemv_n(n, w, r, y, r, C, XQ, ldq, XS, XA, M, NULL, ws, stream);
}

int kt_tern_sum(const float* P, float* y, int R, int M, int sp, void* stream){
  if(M == 0) return 0;
  if(!P || !y || R <= 0 || M < 0 || sp <= 0) return KT_INVALID;
  const long long n = (long long)R * M;
  hipLaunchKernelGGL(k_tern_sum, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, kt_stream(stream), P, y, R, M, sp);
  KT_LAUNCH_CHECK();
  return 0;
}

/* ------------------------------------------------------------------ prefill product */
int kt_tern_gemm(const void* W, int R, int C, const int8_t* XQ, int ldq, const float* XS, const int32_t* XA, int M,
                 float* Y, uint16_t* Y16, int ldy, int32_t* dbg, void* stream){
  (void)XA;                                                  /* signed trits on the matrix cores: no digit offset */
  if(M == 0) return 0;
  if(!W || !XQ || !XS || (!Y && !Y16) || R <= 0 || M < 0 || C <= 0 || C % 128 || ldq < C || ldq % 16 || ldy < R
     || !kt_al(W, 16) || !kt_al(XQ, 16)) return KT_INVALID;
  const int Rp = kt_rp(R), NG = C / 128, ntiles = Rp / KT_TR;
  const uint32_t* codes = (const uint32_t*)W;
  const uint16_t* scales = (const uint16_t*)((const uint8_t*)W + (size_t)Rp * NG * 32);
  const dim3 grid((R + 127) / 128, (M + 127) / 128);
  hipLaunchKernelGGL(k_tern_gemm, grid, dim3(256), 0, kt_stream(stream), codes, scales, R, NG, ntiles, XQ, ldq, XS, M,
                     Y, Y16, ldy, dbg);
  KT_LAUNCH_CHECK();
  return 0;
}

/* ------------------------------------------------------------------ q8_0 */
size_t kt_q8_weight_bytes(int R, int C){
  if(R <= 0 || C <= 0 || C % 32) return 0;
  const size_t Rp = (size_t)kt_rp(R), NB = (size_t)(C / 32);
  return Rp * NB * 32 + Rp * NB * 2;
}

int kt_q8_pack(const uint8_t* rows, int R, int C, void* W, void* stream){
  if(!rows || !W || R <= 0 || C <= 0 || C % 32 || !kt_al(W, 16)) return KT_INVALID;
  const int Rp = kt_rp(R), NB = C / 32;
  uint32_t* codes = (uint32_t*)W;
  uint16_t* scales = (uint16_t*)((uint8_t*)W + (size_t)Rp * NB * 32);
  const long long nw = (long long)Rp * NB * 8;
  hipLaunchKernelGGL(k_q8_pack, dim3((unsigned)((nw + 255) / 256)), dim3(256), 0, kt_stream(stream), rows, R, C, Rp,
                     codes, scales);
  KT_LAUNCH_CHECK();
  return 0;
}

int kt_q8_quant(const float* X, int ldx, int M, int C, int act, int8_t* Q, int ldq, float* D, int ldd, void* stream){
  if(M == 0) return 0;
  if(!X || !Q || !D || M < 0 || C <= 0 || C % 32 || ldx < C || ldq < C || ldd < C / 32) return KT_INVALID;
  const int NB = C / 32;
  hipLaunchKernelGGL(k_quant_q8, dim3((NB + 7) / 8, M), dim3(256), 0, kt_stream(stream), X, ldx, C, act ? 1 : 0, Q,
                     ldq, D, ldd);
  KT_LAUNCH_CHECK();
  return 0;
}

int kt_q8_gemv_splits(int R, int C){
  if(R <= 0 || C <= 0 || C % 32) return 0;
  return kt_nsplit(kt_rp(R) / KT_TR, C / 32, 4);
}

size_t kt_q8_gemv_workspace(int R, int C, int M){
  if(R <= 0 || C <= 0 || C % 32 || M <= 0) return 0;
  const int ntiles = kt_rp(R) / KT_TR;
  return kt_ws_bytes(kt_nsplit(ntiles, C / 32, 4), M, ntiles);
}

int kt_q8_gemv(const void* W, int R, int C, const int8_t* Q, int ldq, const float* D, int ldd, int M, float* Y,
               int ldy, int32_t* dbg, void* ws, void* stream){
  if(M == 0) return 0;
  if(!W || !Q || !D || !Y || R <= 0 || M < 0 || C <= 0 || C % 32 || ldq < C || ldq % 16 || ldd < C / 32 || ldy < R
     || !kt_al(W, 16) || !kt_al(Q, 16)) return KT_INVALID;
  const int Rp = kt_rp(R), NB = C / 32, tiles = Rp / KT_TR;
  KtGemvArgs a = {};
  a.mat[0].codes = (const uint32_t*)W;
  a.mat[0].scales = (const uint16_t*)((const uint8_t*)W + (size_t)Rp * NB * 32);
  a.mat[0].y = Y; a.mat[0].R = R; a.mat[0].ldy = ldy; a.mat[0].tile0 = 0;
  a.nmat = 1; a.NU = NB;
  a.xq = Q; a.ldq = ldq; a.xs = D; a.xa = NULL; a.ldxs = ldd;
  a.M = M; a.dbg = dbg;
  a.nsplit = kt_nsplit(tiles, NB, 4);
  a.Rtot = tiles * KT_TR; a.ntiles = tiles;
  if(kt_ws_set(a, ws)) return KT_INVALID;
  return kt_launch_gemv<KT_FMT_Q8>(a, tiles, kt_stream(stream));
}

/* ------------------------------------------------------------------ MoE */
int kt_moe_topk(const float* logits, int M, int E, int k, int* ids, float* gw, void* stream){
  if(M == 0) return 0;
  if(!logits || !ids || !gw || M < 0 || E <= 0 || E > 1024 || k <= 0 || k > 16 || k > E) return KT_INVALID;
  hipLaunchKernelGGL(k_moe_topk, dim3(M), dim3(64), 0, kt_stream(stream), logits, E, k, ids, gw);
  KT_LAUNCH_CHECK();
  return 0;
}

int kt_moe_sort(const int* ids, int M, int k, int E, int* cnt, int* off, int* xrow, int* where, int* act, int* nact,
                void* stream){
  if(!ids || !cnt || !off || !xrow || !where || !act || !nact || M < 0 || k <= 0 || E <= 0 || E > 1024) return KT_INVALID;
  hipLaunchKernelGGL(k_moe_sort, dim3(1), dim3(1024), 0, kt_stream(stream), ids, M * k, E, cnt, off, xrow, where, act,
                     nact, k);
  KT_LAUNCH_CHECK();
  return 0;
}

int kt_q8_grouped(const void* const* Wexp, int R, int C, int E, const int* cnt, const int* off, const int* act,
                  const int* nact, const int* xrow, int nentries, int M, const int8_t* Q, int ldq,
                  const float* D, int ldd, float* Y, int ldy, int32_t* dbg, void* stream){
  if(nentries == 0) return 0;
  if(!Wexp || !cnt || !off || !act || !nact || !Q || !D || !Y || R <= 0 || C <= 0 || C % 32 || E <= 0
     || nentries < 0 || M <= 0 || ldq < C || ldq % 16 || ldd < C / 32 || ldy < R || !kt_al(Q, 16))
    return KT_INVALID;
  KtGroupedArgs a = {};
  a.wexp = (const uint8_t* const*)Wexp;
  a.R = R; a.C = C; a.NU = C / 32;
  a.cnt = cnt; a.off = off; a.act = act; a.nact = nact; a.xrow = xrow;
  a.xq = Q; a.ldq = ldq; a.xd = D; a.ldd = ldd; a.y = Y; a.ldy = ldy; a.dbg = dbg;
  const int mt = M <= 1 ? 1 : M <= 4 ? 4 : M <= 8 ? 8 : 16;    /* an expert's list holds at most M tokens */
  const int ny = E < nentries ? E : nentries;
  const dim3 grid(kt_rp(R) / KT_TR, ny), block(256);
  hipStream_t s = kt_stream(stream);
  switch(mt){
    case 1: hipLaunchKernelGGL(k_q8_grouped<1>, grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL(k_q8_grouped<4>, grid, block, 0, s, a); break;
    case 8: hipLaunchKernelGGL(k_q8_grouped<8>, grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL(k_q8_grouped<16>, grid, block, 0, s, a); break;
  }
  KT_LAUNCH_CHECK();
  return 0;
}

int kt_moe_combine(const float* yd, const float* ysh, const int* where, const float* gw, int M, int k, int cols,
                   float* x, void* stream){
  if(M == 0) return 0;
  if(!yd || !where || !gw || !x || M < 0 || k <= 0 || cols <= 0) return KT_INVALID;
  hipLaunchKernelGGL(k_moe_combine, dim3(M), dim3(256), 0, kt_stream(stream), yd, ysh, where, gw, k, cols, x);
  KT_LAUNCH_CHECK();
  return 0;
}

}  /* extern "C" */
