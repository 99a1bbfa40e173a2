/* kt_fold.h - arguments of the fused input producers (kt_fold.hip) */
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

struct KtFoldArgs {
  const float* x; int ldx;         /* rmsfold / fold: the row; smfold: a (the SiLU input) */
  const float* r; int ldr;         /* rmsfold: the residual parts (token n's part p at r + n ldr + p C); smfold: b */
  int nparts;                      /* rmsfold: parts to add (0: none) */
  const float* w;                  /* rmsfold: the norm weights [C] */
  const float* sg;                 /* the fold's signs [C] */
  int hd, nk, rep;                 /* smfold: grouped-head order (rep <= 1: none) */
  float* xw; int ldxw;             /* rmsfold: x + parts (nullable) */
  float* xn; int ldxn;             /* rmsfold: the normed row (nullable) */
  float* xo; int ldxo;             /* the folded, scaled row (nullable) */
  int C, HB;
  int8_t* Q; int ldq;              /* int8 row, natural column order */
  float* XS; int32_t* XA;          /* [M][C/128], or [2M][C/128] with hp */
  int hp;                          /* two rows a token: 2n the int8 row, 2n + 1 its residual (ff_q8 tcf.cu:150-205) */
};

hipError_t kt_fold_launch(int mode, const KtFoldArgs& a, int M, hipStream_t s);
