/* kt_common.h - device layouts and shared helpers of the gfx950 quantized linear-layer library.

   Weights are stored per matrix in one buffer: codes, then scales. Rows are padded to a multiple of 8 (a "row
   group", one wave of a decode product; padding rows hold zero weights and scales). The K units (ternary:
   128-column groups; q8_0: 32-column blocks) are taken 8 at a time (a "step": the 8 lanes that share a row take 8
   consecutive units); the last step holds only the units that exist (nc = min(8, NU - 8 s)), so a matrix is
   exactly 32 bytes of codes and 2 bytes of scale per row and unit.

   Ternary ("kt2", 2 bits + 1/8 bit per weight, the reference pack's 2.125 b/w):
     codes  u32 [R8][S][2][nc][8][4]  row group rg, step s, half h (columns 64h .. 64h+63 of a unit), k-lane c,
                                      row r, word j: unit u = 8 s + c, row 8 rg + r, columns 128 u + 64 h + 16 j ..
                                      +15; inside a word, byte b bits 2k..2k+1 hold the digit d = t + 1 in {0,1,2}
                                      of column 16 j + 4 k + b, so (word >> 2k) & 0x03030303 is the digit vector of
                                      four consecutive columns (activation word 4 j + k of the half)
     scales fp16 [R8][NU][8]          per unit and row
   A wave (lane = 8 c + r) reads a (rg, s, h) with one 16-byte load per lane: 1 KB contiguous (full steps).

   q8_0 ("kq8", 8 bits + 1/2 bit per weight, GGUF Q8_0's 1.0625 B/w):
     codes  i8  [R8][S][2][nc][8][16] as above with 32-column units, half h = columns 16 h .. 16 h + 15
     scales fp16 [R8][NU][8]

   Activations are int8 in natural column order, row-major [M][ldq] (ldq a multiple of 16).
   Ternary: XS f32 / XA i32 [M][NG] per 128-column group. q8_0: D f32 [M][ldd] per 32-column block. */
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#define KT_RG 8                       /* rows per row group (one decode wave) */
#define KT_KL 8                       /* lanes along K per row = units per step */
#define KT_MAXMAT 3                   /* matrices sharing one input in a launch (q/k/v, gate/up) */

/* KT_FMT_Q8X / KT_FMT_Q8R: q8_0 weights whose int8 activations are made in the product's own staging from fp32
   rows (kt_q8_quant's numbers, per 32-column unit, so each wave quantizes exactly the units it reads); Q8R applies
   relu^2 first (the MoE down projection's input) */
enum { KT_FMT_TERN = 0, KT_FMT_Q8 = 1, KT_FMT_Q8X = 2, KT_FMT_Q8R = 3 };

/* the one-round-trip decode product (kt_flat.h): slice length and LDS sizes */
#ifndef KT_SL
#define KT_SL 2                       /* steps of a K slice (one register set per step) */
#endif
#define KT_KSMAX 16                   /* waves per block */

template <int FMT, int MT>
struct KtFlat {
  static constexpr int UW = FMT == KT_FMT_TERN ? 128 : 32;   /* bytes of a unit's activations */
  static constexpr int UP = UW + 16;                         /* staged stride (the 8 units of a read on other banks) */
  static constexpr int XW = MT * KT_SL * KT_KL * UP + 16;    /* one wave's staging (+ a dump slot) */
  static size_t lds(int ks){ return (size_t)ks * XW + (size_t)ks * MT * 8 * 4; }
};


__host__ __device__ __forceinline__ int kt_r8(int R){ return (R + KT_RG - 1) / KT_RG; }
__host__ __device__ __forceinline__ int kt_steps(int NU){ return (NU + KT_KL - 1) / KT_KL; }
/* 16-byte index of (row group rg, step s, half h, k-lane c, row r) in a matrix with NU units */
__host__ __device__ __forceinline__ long long kt_widx(int NU, int rg, int s, int h, int c, int r){
  const int nc = NU - s * KT_KL < KT_KL ? NU - s * KT_KL : KT_KL;
  return (long long)rg * NU * 16 + (long long)s * 128 + (h * nc + c) * 8 + r;
}
/* index of the fp16 scale of (rg, unit u, row r) */
__host__ __device__ __forceinline__ long long kt_sidx(int NU, int rg, int u, int r){ return ((long long)rg * NU + u) * 8 + r; }

/* XCD-aware tile order. Workgroups are dispatched to the 8 XCDs round-robin by linear id, and each XCD has its own
   L2. kt_xcd_tile maps the linear id L of a gx x gy grid to a tile (x, y) so that XCD k (the ids L = k mod 8) takes
   a contiguous band of about gx / 8 columns x, walked y-major: the blocks resident on one XCD share their x band's
   data and a few y rows. A bijection of [0, gx gy) for any gx, gy. */
__host__ __device__ __forceinline__ void kt_xcd_tile(int L, int gx, int gy, int& x, int& y){
  const int N = gx * gy, k = L & 7, i = L >> 3;
  const int q = N >> 3, rem = N & 7;
  const int T = k * q + (k < rem ? k : rem) + i;                  /* ids of XCDs before k, then i */
  const int cw = (gx + 7) >> 3, band = T / (cw * gy), w = gx - band * cw < cw ? gx - band * cw : cw;
  const int in = T - band * cw * gy;
  y = in / w;
  x = band * cw + in % w;
}

__device__ __forceinline__ float kt_h2f(uint16_t h){ return __half2float(__ushort_as_half(h)); }

typedef unsigned int kt_u32x4 __attribute__((ext_vector_type(4)));
/* a streaming 128-bit load (each weight byte is read once per product: keep it out of the caches' way; measured on
   MI355X against plain loads, 27B-class step at one token 1.791 -> 1.737 ms; buffer loads with the same bit
   1.733 ms, within the runs' spread, and with the scope bits sc0 / sc1 added no faster) */
__device__ __forceinline__ uint4 kt_ldnt(const uint4* p){
  const kt_u32x4 v = __builtin_nontemporal_load((const kt_u32x4*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

/* global-memory (address space 1) views: pointers read from memory (a plan's tables) are generic to the compiler,
   and generic loads are FLAT instructions, which also count against the LDS wait counter */
#define KT_G __attribute__((address_space(1)))
__device__ __forceinline__ uint4 kt_ldnt_g(const void* p){
  const kt_u32x4 v = __builtin_nontemporal_load((const KT_G kt_u32x4*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
template <typename T>
__device__ __forceinline__ T kt_ldg(const void* p){ return *(const KT_G T*)p; }
__device__ __forceinline__ uint4 kt_ldg4(const void* p){
  const kt_u32x4 v = *(const KT_G kt_u32x4*)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}
template <typename T>
__device__ __forceinline__ void kt_stg(void* p, T v){ *(KT_G T*)p = v; }

__device__ __forceinline__ int kt_dot4(int a, int b, int c){ return __builtin_amdgcn_sdot4(a, b, c, false); }

/* one matrix of a decode launch: its weights, output and the first global row group it owns */
struct KtMat {
  const uint32_t* codes;
  const uint16_t* scales;
  float* y;
  int R, ldy, rg0, pad;
};

#define KT_HP (1 << 30)                /* the hp flag carried in an int argument (tc.cu tc_hp) */

struct KtGemvArgs {
  KtMat mat[KT_MAXMAT];
  int nmat, NU;                       /* matrices; units (groups / blocks) along C */
  int ldq, ldxs;                      /* activation row stride (bytes); xs / xa row stride (units) */
  int M, hp;                          /* input rows; hp: two rows a token (2t: the int8 row, 2t + 1: its residual),
                                         output row t = the fp32 results of rows 2t and 2t + 1 added (tc.cu:405-407) */
};


/* grouped (MoE) launch over the token-sorted lists */
struct KtGroupedArgs {
  const uint8_t* const* wexp;         /* device table: expert e's kq8 buffer */
  int R, C, NU, pad;                  /* rows, columns, blocks */
  const int* cnt; const int* off;     /* per expert: list length and start */
  const int* act; const int* nact;    /* active experts (ascending) and their count */
  const int* xrow;                    /* nullable: input row of list entry p (else p itself) */
  int ldq, ldd, ldy, nrows;           /* nrows: input rows (M with xrow, else the entries) */
  float* y;                           /* output rows [entries][ldy] */
  const float* xf;                    /* Q8X / Q8R: the fp32 input rows [nrows][ldxf] (replace q / d) */
  int ldxf, pad2;
};

/* the value of lane l ^ X (X = 1 .. 32) on the VALU, without the LDS crossbar: DPP quad permutes and mirrors inside a
   row of 16 lanes (l ^ 4 = (l ^ 7) ^ 3, l ^ 8 = (l ^ 15) ^ 7), gfx950's permlane swaps across rows and halves. Every
   DPP source lane is inside the row, so bound_ctrl (zero for an invalid source) never applies; it lets the compiler
   fold the move into the consuming add / max. */
template <int X>
__device__ __forceinline__ int kf_xor(int v){
  if(X == 1) return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true);             /* quad_perm [1,0,3,2] */
  if(X == 2) return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true);             /* quad_perm [2,3,0,1] */
  if(X == 4) return __builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true), 0x1B, 0xF, 0xF,
                                             true);                                 /* half mirror, [3,2,1,0] */
  if(X == 8) return __builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, true), 0x141, 0xF, 0xF,
                                             true);                                 /* mirror, half mirror */
  const int l = __lane_id();
  if(X == 16){
    const auto s = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (l & 16) ? (int)s[0] : (int)s[1];
  }
  const auto s = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return (l & 32) ? (int)s[0] : (int)s[1];
}
template <int X> __device__ __forceinline__ float kf_xorf(float v){ return __int_as_float(kf_xor<X>(__float_as_int(v))); }
template <int X> __device__ __forceinline__ double kf_xord(double v){
  const long long b = __double_as_longlong(v);
  const int lo = kf_xor<X>((int)b), hi = kf_xor<X>((int)(b >> 32));
  return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}
