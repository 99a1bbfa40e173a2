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
