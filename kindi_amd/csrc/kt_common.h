/* kt_common.h - device layouts and shared helpers of the gfx950 quantized linear-layer library.

   Device weight layouts (one buffer per matrix: codes, then scales; rows padded to a multiple of 64):

   Ternary ("kt2", 2 bits + 1/8 bit per weight, the reference pack's 2.125 b/w):
     codes  u32 [Rp/64][NG][2][64][4]     tile of 64 rows, 128-column group g, half h (columns 64h .. 64h+63),
                                          lane l = row (tile * 64 + l), word j = columns 64h + 16j .. +15;
                                          inside a word, byte b bits 2s..2s+1 hold the digit d = t + 1 in {0,1,2}
                                          of column 16j + 4s + b, so (word >> 2s) & 0x03030303 is the digit vector of
                                          four consecutive columns 4s .. 4s+3 (activation word 4j + s)
     scales fp16 [Rp/64][NG][64]          per row and group
   One wave's 16-byte loads for a (tile, group, half) are 1 KB contiguous; a (tile, group) is 2 KB + 128 B.

   q8_0 ("kq8", 8 bits + 1/2 bit per weight, GGUF Q8_0's 1.0625 B/w):
     codes  i8  [Rp/64][NB][2][64][16]    tile, 32-column block b, half h (columns 16h .. 16h+15), lane = row
     scales fp16 [Rp/64][NB][64]

   Activations are int8 in natural column order, row-major [M][ldq] (ldq a multiple of 16).
   Ternary: XS f32 / XA i32 [M][NG] per 128-column group. q8_0: D f32 [M][ldd] per 32-column block. */
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#define KT_TR 64                      /* rows per tile = lanes per wave */
#define KT_WAVES 4                    /* waves per decode block: K slices reduced in LDS */
#ifndef KT_UB_TERN
#define KT_UB_TERN 4                  /* ternary units (128 columns) whose loads a wave keeps in flight */
#endif
#ifndef KT_UB_Q8
#define KT_UB_Q8 8                    /* q8_0 units (32 columns) likewise */
#endif
#ifndef KT_TARGET_WAVES
#define KT_TARGET_WAVES 2048          /* waves a decode launch aims for (K split chosen from it) */
#endif
#ifndef KT_MIN_UNITS
#define KT_MIN_UNITS 2                /* least ternary units per wave when splitting K */
#endif
#define KT_MAXMAT 3                   /* matrices sharing one input in a launch (q/k/v, gate/up) */

enum { KT_FMT_TERN = 0, KT_FMT_Q8 = 1 };

__device__ __forceinline__ float kt_h2f(uint16_t h){ return __half2float(__ushort_as_half(h)); }

typedef unsigned int kt_u32x4 __attribute__((ext_vector_type(4)));
/* a streaming 128-bit load (each weight byte is read once per product: keep it out of the caches' way) */
__device__ __forceinline__ uint4 kt_ldnt(const uint4* p){
  const kt_u32x4 v = __builtin_nontemporal_load((const kt_u32x4*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ int kt_dot4(int a, int b, int c){ return __builtin_amdgcn_sdot4(a, b, c, false); }

/* one matrix of a decode launch: its weights, output and the first global tile index it owns */
struct KtMat {
  const uint32_t* codes;
  const uint16_t* scales;
  float* y;
  int R, ldy, tile0, pad;
};

struct KtGemvArgs {
  KtMat mat[KT_MAXMAT];
  int nmat, NU;                       /* matrices; units (groups / blocks) along C */
  const int8_t* xq; int ldq;          /* activations [M][ldq] */
  const float* xs; const int* xa;     /* per (token, unit): ternary XS / XA; q8_0: D (xa unused) */
  int ldxs;                           /* row stride of xs / xa in units */
  int M;                              /* tokens */
  int32_t* dbg;                       /* nullable: exact unit values [M][R][NU] (single matrix only) */
  float* parts;                       /* [nsplit][M][Rtot] partial sums (nsplit > 1) */
  int* counters;                      /* [npass][ntiles] arrival counters, zero between launches */
  int nsplit, Rtot, ntiles, pad;
};

/* grouped (MoE) launch over the token-sorted lists */
struct KtGroupedArgs {
  const uint8_t* const* wexp;         /* device table: expert e's kq8 buffer */
  int R, C, NU, k;                    /* rows, columns, blocks; routes per token */
  const int* cnt; const int* off;     /* per expert: list length and start */
  const int* act; const int* nact;    /* active experts (ascending) and their count */
  const int* xrow;                    /* nullable: input row of list entry p (else p itself) */
  const int8_t* xq; int ldq;
  const float* xd; int ldd;
  float* y; int ldy;                  /* output row p = list entry p */
  int32_t* dbg;                       /* nullable: [entries][R][NU] */
};
