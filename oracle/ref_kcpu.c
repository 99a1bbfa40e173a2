/* ref_kcpu.c - builds the reference CPU engine's own ternary GEMV (kcpu.c, compiled from where it lies under
   /root/reference) into oracle/_ref/libkcpu_ref.so, and exports it. TEST INFRASTRUCTURE ONLY.
   kcpu.c keeps gemv / rows8 / pair_tables file-static (kcpu.c:79-135); including the file in this translation
   unit and exporting wrappers is the only addition. */
#include KINDI_KCPU_SRC

/* y = W x through the reference's gemv() (kcpu.c:116-135), inside one OpenMP parallel region as kc_step runs it.
   W: pair codes [R/8][C/128][64] u32, S: [R/8][C/128][8] fp32, T: scratch C/2 x 8 floats (32-byte aligned). */
void ref_gemv(const uint8_t* W, const float* S, int R, int C, const float* x, float* y, float* T){
  Model m;
  memset(&m, 0, sizeof(m));
  m.T = T;
  Mat A = {W, S, R, C};
  const Mat* a[1] = {&A};
  float* yy[1] = {y};
  #pragma omp parallel
  gemv(&m, 1, a, yy, x);
}

/* rows8 over 8-row blocks [b0, b1) on the calling thread, with tables built by pair_tables (kcpu.c:79-112) */
void ref_pair_tables(const float* x, float* T, int p0, int p1){ pair_tables(x, T, p0, p1); }
void ref_rows8(const uint8_t* W, const float* S, int R, int C, float* y, const float* T, int b0, int b1){
  Mat A = {W, S, R, C};
  rows8(&A, y, T, b0, b1);
}
