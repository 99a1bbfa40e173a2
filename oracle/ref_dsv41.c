/* ref_dsv41.c - builds the reference's q8_0 CPU arithmetic (dsv41_cpu.c, compiled from where it lies under
   /root/reference, linked with moe_cpu.c, whose MoE functions it calls) into oracle/_ref/libdsv41_ref.so, and exports the file-static activation quantizer and Q8_0
   row-group kernel. TEST INFRASTRUCTURE ONLY. */
#include KINDI_DSV41_SRC

/* quant_q8 (dsv41_cpu.c:251-280): per 32 values, d = fp16(amax / 127) as a float, q = rne(x * 127 / amax) */
void ref_quant_q8(const float* x, int n, int8_t* q, float* d){ quant_q8(x, n, q, d); }

/* k_q8g (dsv41_cpu.c:457-520): 4 Q8_0 rows in the repacked group layout (per block 4 fp16 scales, then 4 x 32
   codes: 136 bytes) x T tokens */
void ref_k_q8g(const uint8_t* w, int nb, int T, const int8_t* xq, const float* xd, int xs, float* y, int ys){
  k_q8g(w, nb, T, xq, xd, xs, y, ys);
}

/* a whole matrix through k_q8g: R / 4 row groups of the repacked layout (nb = C / 32 blocks each), T tokens, the
   groups split over OpenMP threads (this driver is ours; each group's arithmetic is the reference's kernel). Used
   as the q8_0 CPU baseline beside the MoE products. */
void ref_q8_matvec(const uint8_t* g4, int R, int C, int T, const int8_t* xq, const float* xd, float* y, int ys){
  const int nb = C / 32, ng = R / 4;
  #pragma omp parallel for schedule(static)
  for(int g = 0; g < ng; ++g)
    k_q8g(g4 + (size_t)g * nb * 136, nb, T, xq, xd, C, y + (size_t)g * 4, ys);
}
