/* kt_oracle.c - CPU oracle for the quantized linear-layer path. TEST INFRASTRUCTURE ONLY: the parity tests, the
   smoke check and the CPU-baseline leg of bench.py load this library as the checker. Nothing in the product
   (kindi_amd/) may call it.

   Every function restates an algorithm of the reference (ahtx/kindi 0.6.1) from its documented arithmetic; the
   file:line each one follows is given beside it. Integer results (quantized activations, group accumulators,
   routing lists) are exact by construction; floating-point results follow the reference's expression and order
   of operations where one is fixed, and a documented canonical order where the reference's own order depends on
   the launch configuration.

   Canonical fp32 expression of a ternary product (the reference's, tc_hip.cu:171, tc.cu:239-242, chunk.cu:912-913):
     v_g  = sum over the 128 columns of group g of t * q          (exact int32, t in {-1, 0, +1})
     acc  = fmaf((float)v_g, XS[g] * d[g], acc)                    for g = 0, 1, ..., NG-1 in order
   (the reference writes acc += (float)(c - XA) * (XS * d); CUDA and HIP contract that into one fma).

   Canonical fp32 expression of a q8_0 product (lightning.cu:279, dsv41_cpu.c:457-520 per block):
     v_b  = sum over the 32 columns of block b of w * q            (exact int32)
     acc  = fmaf((float)v_b, dw[b] * dx[b], acc)                   for b in order. */
#include <stdint.h>
#include <stddef.h>
#include <string.h>
#include <math.h>
#include <stdlib.h>
#include <immintrin.h>
#include <omp.h>

/* ------------------------------------------------------------------ fp16 <-> fp32 (IEEE binary16, RNE) */
float or_h2f(uint16_t h){
  const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u, m = h & 1023u;
  uint32_t b;
  if(e == 0){
    if(m == 0) b = s;
    else {                                   /* subnormal: m * 2^-24 */
      float f = (float)m * 5.9604644775390625e-8f;
      memcpy(&b, &f, 4);
      b |= s;
    }
  } else if(e == 31) b = s | 0x7F800000u | (m << 13);
  else b = s | ((e + 112u) << 23) | (m << 13);
  float f;
  memcpy(&f, &b, 4);
  return f;
}

uint16_t or_f2h(float f){                    /* round to nearest even, as F16C _cvtss_sh(f, 0) */
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t s = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7FFFFFFFu;
  if(ax >= 0x7F800000u) return (uint16_t)(s | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
  if(ax >= 0x477FF000u) return (uint16_t)(s | 0x7C00u);           /* rounds to >= 65520: inf */
  if(ax < 0x38800000u){                                             /* result subnormal or zero */
    if(ax < 0x33000000u) return (uint16_t)s;                        /* < 2^-25: rounds to 0 */
    const uint32_t e = ax >> 23, m = (ax & 0x7FFFFFu) | 0x800000u;
    const int sh = 126 - (int)e;                                    /* 14 .. 24 */
    uint32_t r = m >> sh;
    const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
    if(rem > half || (rem == half && (r & 1u))) ++r;
    return (uint16_t)(s | r);
  }
  uint32_t r = ((ax >> 13) - (112u << 10));
  const uint32_t rem = ax & 0x1FFFu;
  if(rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
  return (uint16_t)(s | r);
}

/* ------------------------------------------------------------------ int8 activations, 128-column groups
   Follows k_tc_q8 (tc_hip.cu:43-74) and tcq128 (tc.cu:160-194): amax = max |x| over the group, id = 127 / amax
   (0 when amax = 0), q = round-to-nearest-even(x * id), XS = amax / 127, XA = sum q.
   per_row = 1: the BASELINE configs' per-token absmax: amax over the whole row, the same XS for every group of the
   row (the formula is unchanged); XA stays per group. Q is [M][ldq] int8 in natural column order.
   per_row = 2 / 3 (hp: two rows a token, Q / XS / XA with 2M rows): row 2n is the per-group row above; row 2n + 1
   quantizes the residual r = fma(-q, amax / 127, x) (the reference's compiler contracts x - q (amax / 127) into one
   fma) at a fixed amax:
     2: k_tc_q8 with hp (tc.cu:195-209, tcq128 tc.cu:160-194): a2 = amax / 254, q2 = clamp(rne(r (127 / a2)), -127,
        127), XS = a2 / 127;
     3: the producers' ff_q8 with hp (tcf.cu:150-205): q2 = clamp(rne(r (32258 / amax)), -127, 127), XS = amax / 32258.
   XA = the sum of the row's q2. Both residual scales are 0 when amax = 0 (every q2 is then 0). */
static int or_clamp127(int q){ return q < -127 ? -127 : (q > 127 ? 127 : q); }

void or_quant_q8(const float* X, int ldx, int M, int C, int per_row, int8_t* Q, int ldq, float* XS, int* XA){
  const int NG = C / 128, hp = per_row >= 2;
  for(int n = 0; n < M; ++n){
    const float* x = X + (size_t)n * ldx;
    const size_t n0 = hp ? 2 * (size_t)n : (size_t)n;
    float rmax = 0.0f;
    if(per_row == 1) for(int c = 0; c < C; ++c) rmax = fmaxf(rmax, fabsf(x[c]));
    for(int g = 0; g < NG; ++g){
      float amax = rmax;
      if(per_row != 1){
        amax = 0.0f;
        for(int e = 0; e < 128; ++e) amax = fmaxf(amax, fabsf(x[g * 128 + e]));
      }
      const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
      int sum = 0, sum2 = 0;
      const float sc = amax / 127.0f, a2 = amax / 254.0f;
      const float id2 = per_row == 2 ? (a2 != 0.0f ? 127.0f / a2 : 0.0f) : (amax != 0.0f ? 32258.0f / amax : 0.0f);
      for(int e = 0; e < 128; ++e){
        const int q = (int)nearbyintf(x[g * 128 + e] * id);
        Q[n0 * ldq + g * 128 + e] = (int8_t)q;
        sum += q;
        if(hp){
          const float r = fmaf(-(float)q, sc, x[g * 128 + e]);
          const int q2 = or_clamp127((int)nearbyintf(r * id2));
          Q[(n0 + 1) * ldq + g * 128 + e] = (int8_t)q2;
          sum2 += q2;
        }
      }
      XS[n0 * NG + g] = sc;
      XA[n0 * NG + g] = sum;
      if(hp){
        XS[(n0 + 1) * NG + g] = per_row == 2 ? a2 / 127.0f : amax / 32258.0f;
        XA[(n0 + 1) * NG + g] = sum2;
      }
    }
  }
}

/* ------------------------------------------------------------------ ternary products
   Weights in the reference pack format (convert.py:1-11, 49-52, 144-159): bcodes [C/4][R], byte s of row r =
   t0 + 3 t1 + 9 t2 + 27 t3 (digits d in {0,1,2} of columns 4s .. 4s+3, weight = (d - 1) * scale); scales dpm
   [C/128][R] fp16 bits. */
/* acc[n][r][g] = sum_{c in g} t(r, c) * Q[n][c]: the exact int32 group value (tc_hip.cu:12-15: sum (d-1) q =
   sum d q - XA). Rows in parallel; each row's trits are decoded once. */
void or_tern_acc(const uint8_t* bcodes, int R, int C, const int8_t* Q, int ldq, int M, int32_t* acc){
  const int NG = C / 128;
  #pragma omp parallel
  {
    int8_t* t = (int8_t*)malloc((size_t)C);
    #pragma omp for schedule(static)
    for(int r = 0; r < R; ++r){
      for(int s = 0; s < C / 4; ++s){
        unsigned int b = bcodes[(size_t)s * R + r];
        for(int i = 0; i < 4; ++i){ t[4 * s + i] = (int8_t)((int)(b % 3u) - 1); b /= 3u; }
      }
      for(int n = 0; n < M; ++n){
        const int8_t* q = Q + (size_t)n * ldq;
        for(int g = 0; g < NG; ++g){
          int v = 0;
          for(int e = 0; e < 128; ++e) v += t[g * 128 + e] * q[g * 128 + e];
          acc[((size_t)n * R + r) * NG + g] = v;
        }
      }
    }
    free(t);
  }
}

/* Y[n][r] (ldy) from the group values: the canonical expression above, groups in order. */
void or_tern_out(const int32_t* acc, const float* XS, const uint16_t* dpm, int R, int NG, int M, float* Y, int ldy){
  for(int n = 0; n < M; ++n)
    for(int r = 0; r < R; ++r){
      float a = 0.0f;
      for(int g = 0; g < NG; ++g){
        const float d = or_h2f(dpm[(size_t)g * R + r]);
        a = fmaf((float)acc[((size_t)n * R + r) * NG + g], XS[(size_t)n * NG + g] * d, a);
      }
      Y[(size_t)n * ldy + r] = a;
    }
}

/* The prefill product's order for per-row activation scales (one XS per token, kt_quant_q8 per_row): the weight
   scale alone goes into the group chain, a = fmaf((float)v_g, d_g, a) over g in order, and the token's scale
   multiplies the sum once: Y = a * XS[n][0]. The same real value as or_tern_out when XS[n][g] does not depend on g;
   only the fp32 rounding order differs. */
void or_tern_out_rs(const int32_t* acc, const float* XS, const uint16_t* dpm, int R, int NG, int M, float* Y, int ldy){
  for(int n = 0; n < M; ++n)
    for(int r = 0; r < R; ++r){
      float a = 0.0f;
      for(int g = 0; g < NG; ++g)
        a = fmaf((float)acc[((size_t)n * R + r) * NG + g], or_h2f(dpm[(size_t)g * R + r]), a);
      Y[(size_t)n * ldy + r] = a * XS[(size_t)n * NG];
    }
}

/* The same sums added in a fixed tree: the K units split into nsplit contiguous ranges, each range into nwave
   contiguous slices (slice bounds floor(i * n / parts)); a slice is a sequential fma chain from 0, the slices of a
   range are added left to right, then the ranges left to right. nsplit = nwave = 1 is or_tern_out itself. This is
   the summation order of a K-split decode product (k_tc_mv with splits + k_tc_sum, tc_hip.cu:180-199, 271-279, is
   the case nwave = 1). fmt 0: ternary (scale XS[g] * d), fmt 1: q8_0 (scale d * D[b]); dq: scales as fp32. */
static float or_chain(const int32_t* v, const float* xs, const float* d, int fmt, int a, int b){
  float s = 0.0f;
  for(int u = a; u < b; ++u) s = fmaf((float)v[u], fmt == 0 ? xs[u] * d[u] : d[u] * xs[u], s);
  return s;
}
void or_out_tree(const int32_t* acc, const float* XS, int ldxs, const float* dq, int R, int NU, int M, int nsplit,
                 int nwave, int fmt, float* Y, int ldy){
  float* d = (float*)malloc((size_t)NU * sizeof(float));
  for(int n = 0; n < M; ++n)
    for(int r = 0; r < R; ++r){
      for(int u = 0; u < NU; ++u) d[u] = dq[(size_t)u * R + r];
      const int32_t* v = acc + ((size_t)n * R + r) * NU;
      const float* xs = XS + (size_t)n * ldxs;
      float y = 0.0f;
      for(int sp = 0; sp < nsplit; ++sp){
        const int u0 = (int)((long long)sp * NU / nsplit), u1 = (int)((long long)(sp + 1) * NU / nsplit);
        float q = 0.0f;
        for(int w = 0; w < nwave; ++w){
          const int a = u0 + (int)((long long)w * (u1 - u0) / nwave), b = u0 + (int)((long long)(w + 1) * (u1 - u0) / nwave);
          const float p = or_chain(v, xs, d, fmt, a, b);
          q = w == 0 ? p : q + p;
        }
        y = sp == 0 ? q : y + q;
      }
      Y[(size_t)n * ldy + r] = y;
    }
  free(d);
}

/* The decode products' order: the K units of a row are taken KL at a time (steps), the steps split into KS
   contiguous slices (slice k = steps [k S / KS, (k + 1) S / KS)); in a slice, lane c chains fmaf over its units
   st KL + c in increasing step order, the KL lane sums are added by an xor butterfly (level k adds the lanes c and
   c ^ 2^k; KL = 8: ((l0 + l1) + (l2 + l3)) + ((l4 + l5) + (l6 + l7))), and the slice sums are added left to right.
   fmt and dq as or_out_tree. */
void or_out_lanes(const int32_t* acc, const float* XS, int ldxs, const float* dq, int R, int NU, int M, int KL, int KS,
                  int fmt, float* Y, int ldy){
  float* d = (float*)malloc((size_t)NU * sizeof(float));
  float lane[64], nxt[64];
  for(int n = 0; n < M; ++n)
    for(int r = 0; r < R; ++r){
      for(int u = 0; u < NU; ++u) d[u] = dq[(size_t)u * R + r];
      const int32_t* v = acc + ((size_t)n * R + r) * NU;
      const float* xs = XS + (size_t)n * ldxs;
      const int S = (NU + KL - 1) / KL;
      float y = 0.0f;
      for(int k = 0; k < KS; ++k){
        const int s0 = k * S / KS, s1 = (k + 1) * S / KS;
        for(int c = 0; c < KL; ++c){
          float s = 0.0f;
          for(int st = s0; st < s1; ++st){
            const int u = st * KL + c;
            if(u < NU) s = fmaf((float)v[u], fmt == 0 ? xs[u] * d[u] : d[u] * xs[u], s);
          }
          lane[c] = s;
        }
        for(int st = 1; st < KL; st *= 2){
          for(int c = 0; c < KL; ++c) nxt[c] = lane[c] + lane[c ^ st];
          for(int c = 0; c < KL; ++c) lane[c] = nxt[c];
        }
        y = k == 0 ? lane[0] : y + lane[0];
      }
      Y[(size_t)n * ldy + r] = y;
    }
  free(d);
}

/* k_tc_sum (tc_hip.cu:271-279): y[n][r] = sum over parts p = 0 .. sp-1 of P[(n sp + p) R + r], in part order */
void or_tern_sum(const float* P, float* y, int R, int M, int sp){
  for(int n = 0; n < M; ++n)
    for(int r = 0; r < R; ++r){
      const float* q = P + (size_t)n * sp * R + r;
      float s = q[0];
      for(int p = 1; p < sp; ++p) s += q[(size_t)p * R];
      y[(size_t)n * R + r] = s;
    }
}

/* ------------------------------------------------------------------ the CPU engine's fp32 pair-table GEMV
   Restated from kcpu.c:72-135 (pair_tables 79-86, rows8 87-112, gemv 116-135) with the pair-code layout of
   cpu.paircodes (cpu.py:69-88): W [R/8][C/128][64] u32, word p = the 8 rows' 4-bit codes of columns 2p, 2p+1
   (code k < 8 selects one of the 8 nonzero (w0, w1) pairs, code 8 = both zero); S [R/8][C/128][8] fp32.
   Per call: a table of the 8 pair sums per column pair; per 8-row block and group, two vector partial sums over
   the even / odd pairs, added, then fmadd with the 8 rows' scales. No activation quantization. */
static void or_pair_tables(const float* x, float* T, int p0, int p1){
  for(int p = p0; p < p1; ++p){
    const float x0 = x[2 * p], x1 = x[2 * p + 1];
    float* t = T + (size_t)p * 8;
    t[0] = -x0 - x1; t[1] = -x1; t[2] = x0 - x1; t[3] = -x0;
    t[4] = x0; t[5] = -x0 + x1; t[6] = x1; t[7] = x0 + x1;
  }
}

static void or_rows8(const uint32_t* P, const float* S, int C, float* y, const float* T, int b0, int b1){
  const int G = C / 128;
  const __m256i sh = _mm256_setr_epi32(0, 4, 8, 12, 16, 20, 24, 28);
  const __m256i f = _mm256_set1_epi32(15);
  for(int rb = b0; rb < b1; ++rb){
    __m256 acc = _mm256_setzero_ps();
    for(int g = 0; g < G; ++g){
      const uint32_t* pw = P + ((size_t)rb * G + g) * 64;
      const float* pt = T + (size_t)g * 64 * 8;
      __m256 s0 = _mm256_setzero_ps(), s1 = s0;
      for(int p = 0; p < 64; p += 2){
        const __m256i c0 = _mm256_and_si256(_mm256_srlv_epi32(_mm256_set1_epi32((int)pw[p]), sh), f);
        const __m256i c1 = _mm256_and_si256(_mm256_srlv_epi32(_mm256_set1_epi32((int)pw[p + 1]), sh), f);
        const __m256 v0 = _mm256_permutevar8x32_ps(_mm256_load_ps(pt + 8 * p), c0);
        const __m256 v1 = _mm256_permutevar8x32_ps(_mm256_load_ps(pt + 8 * p + 8), c1);
        const __m256 z0 = _mm256_castsi256_ps(_mm256_cmpeq_epi32(c0, _mm256_set1_epi32(8)));
        const __m256 z1 = _mm256_castsi256_ps(_mm256_cmpeq_epi32(c1, _mm256_set1_epi32(8)));
        s0 = _mm256_add_ps(s0, _mm256_andnot_ps(z0, v0));
        s1 = _mm256_add_ps(s1, _mm256_andnot_ps(z1, v1));
      }
      acc = _mm256_fmadd_ps(_mm256_add_ps(s0, s1), _mm256_loadu_ps(S + ((size_t)rb * G + g) * 8), acc);
    }
    _mm256_storeu_ps(y + (size_t)rb * 8, acc);
  }
}

/* cpu.paircodes (cpu.py:69-88) from the pack: P [R/8][C/128][64] u32, word p = the 8 rows' 4-bit codes of columns
   2p, 2p+1 (code of the digit pair (d0, d1): d0 + 3 d1 mapped 0 1 2 3 8 4 5 6 7, i.e. 4 = both zero -> 8) */
void or_paircodes(const uint8_t* bcodes, int R, int C, uint32_t* P){
  static const uint32_t code[9] = {0, 1, 2, 3, 8, 4, 5, 6, 7};
  const int G = C / 128;
  #pragma omp parallel for schedule(static)
  for(int rb = 0; rb < R / 8; ++rb)
    for(int g = 0; g < G; ++g)
      for(int p = 0; p < 64; ++p){
        const int s = (g * 128 + 2 * p) >> 2, sh = (2 * p) & 3;      /* both columns sit in one pack byte */
        uint32_t w = 0;
        for(int l = 0; l < 8; ++l){
          unsigned int b = bcodes[(size_t)s * R + rb * 8 + l];
          if(sh) b /= 9u;
          const uint32_t d0 = b % 3u, d1 = (b / 3u) % 3u;
          w |= code[d0 + 3 * d1] << (4 * l);
        }
        P[((size_t)rb * G + g) * 64 + p] = w;
      }
}

/* y = W x over all threads: tables for the whole input, then 8-row blocks split evenly (kcpu.c:116-135).
   T: scratch of C * 4 floats (C/2 pairs x 8), 32-byte aligned. */
void or_pair_gemv(const uint32_t* P, const float* S, int R, int C, const float* x, float* y, float* T){
  #pragma omp parallel
  {
    const int nt = omp_get_num_threads(), id = omp_get_thread_num();
    const long long np = C / 2, nb = R / 8;
    or_pair_tables(x, T, (int)(np * id / nt), (int)(np * (id + 1) / nt));
    #pragma omp barrier
    or_rows8(P, S, C, y, T, (int)(nb * id / nt), (int)(nb * (id + 1) / nt));
  }
}

/* ------------------------------------------------------------------ q8_0
   Weights: GGUF Q8_0 rows, blocks of 34 bytes (fp16 scale, 32 int8), as dsv41_cpu.c:77-78 (QK, BQ8).
   Activations: quant_q8 (dsv41_cpu.c:251-280, moe_cpu.c:84-112): per block of 32, d = fp16(amax / 127) kept as a
   float, q = round-to-nearest-even(x * (127 / amax)) (0 when amax = 0). */
void or_q8_quant(const float* x, int n, int8_t* q, float* d){
  for(int b = 0; b < n / 32; ++b){
    float amax = 0.0f;
    for(int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[b * 32 + j]));
    d[b] = or_h2f(or_f2h(amax / 127.0f));
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    for(int j = 0; j < 32; ++j) q[b * 32 + j] = (int8_t)(int)nearbyintf(x[b * 32 + j] * id);
  }
}

/* exact per-block values acc[n][r][b] = sum w * q (rows R, C columns, M tokens; token n's row is Q + n ldq) */
void or_q8_acc(const uint8_t* blocks, int R, int C, const int8_t* Q, int ldq, int M, int32_t* acc){
  const int nb = C / 32;
  #pragma omp parallel for schedule(static)
  for(int r = 0; r < R; ++r)
    for(int n = 0; n < M; ++n)
      for(int b = 0; b < nb; ++b){
        const int8_t* w = (const int8_t*)(blocks + ((size_t)r * nb + b) * 34 + 2);
        const int8_t* q = Q + (size_t)n * ldq + b * 32;
        int v = 0;
        for(int j = 0; j < 32; ++j) v += w[j] * q[j];
        acc[((size_t)n * R + r) * nb + b] = v;
      }
}

/* Y[n][r] = canonical fp32 expression of the q8_0 product from the exact block values; D = activation scales
   [M][ldd] */
void or_q8_out(const int32_t* acc, const uint8_t* blocks, int R, int C, const float* D, int ldd, int M, float* Y, int ldy){
  const int nb = C / 32;
  for(int n = 0; n < M; ++n)
    for(int r = 0; r < R; ++r){
      float a = 0.0f;
      for(int b = 0; b < nb; ++b){
        uint16_t h;
        memcpy(&h, blocks + ((size_t)r * nb + b) * 34, 2);
        a = fmaf((float)acc[((size_t)n * R + r) * nb + b], or_h2f(h) * D[(size_t)n * ldd + b], a);
      }
      Y[(size_t)n * ldy + r] = a;
    }
}

/* AVX2 q8_0 GEMV for the CPU baseline: per block maddubs + madd (an exact int32 dot, as dsv41_cpu.c:452-520),
   fp32 fma with both scales; rows over all threads. One token. */
void or_q8_gemv_avx2(const uint8_t* blocks, int R, int C, const int8_t* q, const float* d, float* y){
  const int nb = C / 32;
  #pragma omp parallel for schedule(static)
  for(int r = 0; r < R; ++r){
    const __m256i ones = _mm256_set1_epi16(1);
    __m256 acc = _mm256_setzero_ps();
    const uint8_t* row = blocks + (size_t)r * nb * 34;
    for(int b = 0; b < nb; ++b){
      uint16_t h;
      memcpy(&h, row + b * 34, 2);
      const __m256i w = _mm256_loadu_si256((const __m256i*)(row + b * 34 + 2));
      const __m256i x = _mm256_loadu_si256((const __m256i*)(q + b * 32));
      const __m256i s = _mm256_madd_epi16(_mm256_maddubs_epi16(_mm256_sign_epi8(w, w), _mm256_sign_epi8(x, w)), ones);
      acc = _mm256_fmadd_ps(_mm256_cvtepi32_ps(s), _mm256_set1_ps(or_h2f(h) * d[b]), acc);
    }
    __m128 v = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    v = _mm_add_ps(v, _mm_movehl_ps(v, v));
    v = _mm_add_ss(v, _mm_movehdup_ps(v));
    y[r] = _mm_cvtss_f32(v);
  }
}

/* ------------------------------------------------------------------ MoE routing lists and combine
   lt_moe_lists (lightning.cu:1318-1349): cnt[e] = tokens of expert e, off[e] = exclusive prefix sum in expert
   order, xrow[p] = the token of list entry p, where[t k + j] = the entry of (t, j). The reference fills an
   expert's range in atomic order ("the order of the tokens inside an expert's range does not change any
   number"); the canonical order here is ascending flat index t k + j (a stable sort). */
void or_moe_sort(const int* ids, int M, int k, int E, int* cnt, int* off, int* xrow, int* where){
  for(int e = 0; e < E; ++e) cnt[e] = 0;
  for(int i = 0; i < M * k; ++i) cnt[ids[i]]++;
  int o = 0;
  for(int e = 0; e < E; ++e){ off[e] = o; o += cnt[e]; }
  int* fill = (int*)calloc((size_t)(E > 0 ? E : 1), sizeof(int));
  for(int i = 0; i < M * k; ++i){
    const int e = ids[i], p = off[e] + fill[e]++;
    xrow[p] = i / k;
    where[i] = p;
  }
  free(fill);
}

/* lt_moe_combine (lightning.cu:1352-1361): x[t][i] += sum_j gw[t k + j] * yd[where[t k + j]][i] (+ ysh[t][i]);
   the j-sum in selection order from 0, each term one fma (the reference's s += g * y, contracted). */
void or_moe_combine(const float* yd, const float* ysh, const int* where, const float* gw, int M, int k, int cols, float* x){
  for(int t = 0; t < M; ++t)
    for(int i = 0; i < cols; ++i){
      float s = 0.0f;
      for(int j = 0; j < k; ++j) s = fmaf(gw[t * k + j], yd[(size_t)where[t * k + j] * cols + i], s);
      x[(size_t)t * cols + i] += ysh ? s + ysh[(size_t)t * cols + i] : s;
    }
}

/* Router as the BASELINE config states it: softmax over E logits, the k largest probabilities, weights = the
   chosen probabilities divided by their sum. (The reference's Lightning router is sigmoid + bias,
   lightning.cu:348-468; the benchmark config names softmax.) Computed in the equivalent form that needs no full
   softmax: the softmax is monotone in the logit, so the k largest logits are chosen (ties: lower expert index), and
   p_j / sum over the chosen p_i = exp(l_j - l_max) / sum over the chosen exp(l_i - l_max) (the denominator of the
   full softmax cancels). fp32 with expf, the sum in selection order. */
/* a ranks above b: numbers by value, NaN below every number (never chosen before a number); equal values do not rank
   above each other, so the scan keeps the lower index */
static int or_above(float a, float b){
  if(a != a) return 0;
  if(b != b) return 1;
  return a > b;
}
/* the k best of v[0 .. E-1] by or_above, ties to the lower index, into ids */
static void or_pick(const float* v, int E, int k, int* ids){
  for(int j = 0; j < k; ++j){
    int best = -1;
    for(int e = 0; e < E; ++e){
      int used = 0;
      for(int i = 0; i < j; ++i) if(ids[i] == e) used = 1;
      if(!used && (best < 0 || or_above(v[e], v[best]))) best = e;
    }
    ids[j] = best;
  }
}
void or_router_topk(const float* logits, int M, int E, int k, int* ids, float* gw){
  for(int t = 0; t < M; ++t){
    const float* l = logits + (size_t)t * E;
    or_pick(l, E, k, ids + (size_t)t * k);
    float p[64], s = 0.0f;
    for(int j = 0; j < k; ++j){ p[j] = expf(l[ids[t * k + j]] - l[ids[t * k]]); s += p[j]; }
    for(int j = 0; j < k; ++j) gw[t * k + j] = p[j] / s;
  }
}

/* Kindi's Lightning router (lt_topk, lightning.cu:373-412; lt_router_topk 414-468): score s_e = 1 / (1 + exp(-l_e)),
   choice s_e + bias[e], the k largest choices (ties to the lower index), weights s_j / tot * scale with tot the sum of
   the chosen scores in pick order. fp32 with expf (the reference's __expf is its fast approximation). */
void or_router_sig(const float* logits, const float* bias, float scale, int M, int E, int k, int* ids, float* gw){
  float* sc = (float*)malloc(sizeof(float) * (size_t)E);
  float* ch = (float*)malloc(sizeof(float) * (size_t)E);
  for(int t = 0; t < M; ++t){
    const float* l = logits + (size_t)t * E;
    for(int e = 0; e < E; ++e){
      sc[e] = 1.0f / (1.0f + expf(-l[e]));
      ch[e] = sc[e] + bias[e];
    }
    int* id = ids + (size_t)t * k;
    or_pick(ch, E, k, id);
    float tot = 0.0f;
    for(int j = 0; j < k; ++j) tot += sc[id[j]];
    for(int j = 0; j < k; ++j) gw[(size_t)t * k + j] = sc[id[j]] / tot * scale;
  }
  free(sc);
  free(ch);
}

/* ------------------------------------------------------------------ fused producers of a product's input
   k_rmsfold_qT / k_fold_fwht_qT / k_smfold_qT (tcf.cu:370-426; the numbers of k_rmsfold kindi.cu:350-394 and the
   fast forms ff_rmsfold / ff_fold / ff_smfold tcf.cu:218-312, which are bit-identical to them). Per token row:
     rmsfold: xf = x + (r_0 + r_1 + ... + r_{n-1})          parts summed in part order (rsum kindi.cu:344-348)
              s  = 1 / sqrt((float)(S / C) + 1e-6)            S: the double sum of squares in the reference's order
              xn = (xf * s) * w;  v = sg * xn
     fold:    v = sg * x
     smfold:  v = sg[e] * ((a / (1 + exp(-a))) * b) at the permuted source column (tcf.cu:284-291)
   then v goes through the unnormalised Walsh-Hadamard transform of each HB-column block (stages h = 1, 2, 4, ... in
   order, pair (i, i + h) -> (a + b, a - b): fwht_chunks / fwht_n kindi.cu:91-116, ff_fwht tcf.cu:60-96), is scaled by
   1/sqrt(HB) (the fp32 constant 0.044194173824159220878 for HB = 512, exactly 2^-5 / 2^-6 for 1024 / 4096,
   ff_scale_store tcf.cu:98-104), stored as xo, and quantized to int8 per 128-column group with k_tc_q8's numbers
   (or_quant_q8 above; ff_q8_row tcf.cu:106-150).
   The double sum of squares: thread j of 512 adds (double)xf[j + 512 m]^2 for m = 0, 1, ... in order; each warp of
   32 threads combines by the xor butterfly (offsets 16, 8, 4, 2, 1: wsum_d kindi.cu:81-84); warp 0 takes the 16 warp
   sums (lanes 16..31 zero) through the same butterfly (kindi.cu:367-373). */
static double or_bfly32(double* a){
  double b[32];
  for(int o = 16; o > 0; o >>= 1){
    for(int l = 0; l < 32; ++l) b[l] = a[l] + a[l ^ o];
    memcpy(a, b, sizeof(b));
  }
  return a[0];
}

double or_sumsq(const float* xf, int C){
  double warp[32], red[32];
  for(int w = 0; w < 16; ++w){
    for(int l = 0; l < 32; ++l){
      const int j = 32 * w + l;
      double acc = 0.0;
      for(int e = j; e < C; e += 512){ const double d = (double)xf[e]; acc += d * d; }
      warp[l] = acc;
    }
    red[w] = or_bfly32(warp);
  }
  for(int l = 16; l < 32; ++l) red[l] = 0.0;
  return or_bfly32(red);
}

static float or_fold_scale(int HB){
  return HB == 512 ? 0.044194173824159220878f : (float)(1.0 / sqrt((double)HB));
}

/* in place: the unnormalised transform of each HB block of v[0..C), then the scale */
void or_fwht_blocks(float* v, int C, int HB){
  const float sc = or_fold_scale(HB);
  for(int b0 = 0; b0 < C; b0 += HB){
    float* u = v + b0;
    for(int h = 1; h < HB; h <<= 1)
      for(int i = 0; i < HB; ++i)
        if(!(i & h)){ const float a = u[i], b = u[i + h]; u[i] = a + b; u[i + h] = a - b; }
  }
  for(int e = 0; e < C; ++e) v[e] = v[e] * sc;
}

/* r: token n's parts at r + n ldr + p C (the parts of a column-split product, C apart, tc.cu:403) */
void or_rmsfold_q8(const float* x, int ldx, const float* r, int ldr, int nparts, const float* w, const float* sg,
                   int M, int C, int HB, float* xw, int ldxw, float* xn, int ldxn, float* xo, int ldxo,
                   int8_t* Q, int ldq, float* XS, int* XA){
  const int hp = (HB >> 30) & 1;                 /* HB | 1 << 30: two int8 rows a token (ff_q8 hp) */
  HB &= ~(1 << 30);
  float* xf = (float*)malloc(sizeof(float) * C);
  float* v = (float*)malloc(sizeof(float) * C);
  for(int n = 0; n < M; ++n){
    for(int e = 0; e < C; ++e){
      float f = x[(size_t)n * ldx + e];
      if(nparts > 0){
        const float* rn = r + (size_t)n * ldr;
        float rv = rn[e];
        for(int p = 1; p < nparts; ++p) rv += rn[(size_t)p * C + e];
        f = f + rv;
      }
      xf[e] = f;
    }
    const double S = or_sumsq(xf, C);
    const float s = 1.0f / sqrtf((float)(S / C) + 1e-6f);
    for(int e = 0; e < C; ++e){
      const float nv = (xf[e] * s) * w[e];
      if(nparts > 0 && xw) xw[(size_t)n * ldxw + e] = xf[e];
      if(xn) xn[(size_t)n * ldxn + e] = nv;
      v[e] = sg[e] * nv;
    }
    or_fwht_blocks(v, C, HB);
    if(xo) memcpy(xo + (size_t)n * ldxo, v, sizeof(float) * C);
    const size_t n0 = hp ? 2 * (size_t)n : (size_t)n;
    or_quant_q8(v, C, 1, C, hp ? 3 : 0, Q + n0 * ldq, ldq, XS + n0 * (C / 128), XA + n0 * (C / 128));
  }
  free(xf); free(v);
}

void or_fold_q8(const float* x, int ldx, const float* sg, int M, int C, int HB, float* xo, int ldxo,
                int8_t* Q, int ldq, float* XS, int* XA){
  const int hp = (HB >> 30) & 1;                 /* HB | 1 << 30: two int8 rows a token (ff_q8 hp) */
  HB &= ~(1 << 30);
  float* v = (float*)malloc(sizeof(float) * C);
  for(int n = 0; n < M; ++n){
    for(int e = 0; e < C; ++e) v[e] = sg[e] * x[(size_t)n * ldx + e];
    or_fwht_blocks(v, C, HB);
    if(xo) memcpy(xo + (size_t)n * ldxo, v, sizeof(float) * C);
    const size_t n0 = hp ? 2 * (size_t)n : (size_t)n;
    or_quant_q8(v, C, 1, C, hp ? 3 : 0, Q + n0 * ldq, ldq, XS + n0 * (C / 128), XA + n0 * (C / 128));
  }
  free(v);
}

/* the source column of output column e under the grouped-head order (tcf.cu:284-289; perm_rep <= 1: none) */
int or_perm_src(int e, int hd, int nk, int rep){
  if(rep <= 1) return e;
  const int h = e % hd, g = e / hd, rp = g % rep, k = g / rep;
  return h + hd * (k + nk * rp);
}

void or_smfold_q8(const float* a, int lda, const float* b, int ldb, const float* sg, int hd, int nk, int rep,
                  int M, int C, int HB, float* xo, int ldxo, int8_t* Q, int ldq, float* XS, int* XA){
  const int hp = (HB >> 30) & 1;                 /* HB | 1 << 30: two int8 rows a token (ff_q8 hp) */
  HB &= ~(1 << 30);
  float* v = (float*)malloc(sizeof(float) * C);
  for(int n = 0; n < M; ++n){
    for(int e = 0; e < C; ++e){
      const int src = or_perm_src(e, hd, nk, rep);
      const float xa = a[(size_t)n * lda + src];
      const float m = (xa / (1.0f + expf(-xa))) * b[(size_t)n * ldb + src];
      v[e] = sg[e] * m;
    }
    or_fwht_blocks(v, C, HB);
    if(xo) memcpy(xo + (size_t)n * ldxo, v, sizeof(float) * C);
    const size_t n0 = hp ? 2 * (size_t)n : (size_t)n;
    or_quant_q8(v, C, 1, C, hp ? 3 : 0, Q + n0 * ldq, ldq, XS + n0 * (C / 128), XA + n0 * (C / 128));
  }
  free(v);
}
