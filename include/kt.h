/* kt.h - C ABI of libkt_gfx950.so, the MI355X (gfx950) kernel library for Kindi's quantized linear layer.

   It replaces the kernel module Kindi compiles at run time (cp.RawModule over kindi.cu + tc_hip.cu + ...,
   spec.py:144-151, 187-195; engine.py:88-92) and launches through gpudrv.driver() (gpudrv.py:24-101): a prebuilt
   shared library, loaded with ctypes, exporting host launchers with plain pointers and sizes.

   Conventions (all entry points):
   - every pointer argument is a device pointer owned by the caller (as Kindi's CuPy buffers, engine.py:193-204,
     spec.py:523-593); the library never allocates, frees or synchronizes. Its only device state is the fixed
     workspace array of kt_moe_decode_noalloc (4 MiB a GPU, held until the process ends); every other entry point
     works on caller buffers alone;
   - `stream` is a hipStream_t (NULL = the null stream); launches are asynchronous and graph-capturable;
   - the return value is a hipError_t as int: 0 on success, hipErrorInvalidValue (1) for a shape, stride or
     alignment the kernels do not take (Kindi raises SystemExit / RuntimeError there: spec.py:195-196,
     layout.py:38-39, tp.py:944-945), else the launch error;
   - M = 0 tokens is a no-op returning 0;
   - between kt_record_begin and kt_record_end, the calling thread's launchers record their launches instead of
     launching them (launch records, below).

   Numbers (the reference's, tc.cu:1-18, tc_hip.cu:8-15): activations are int8 per 128-column group (XS = amax/127,
   q = round-to-nearest-even(x * 127 / amax), XA = sum q); a group's value v = sum t q over its 128 columns is an
   exact int32 (t in {-1, 0, +1}); the fp32 output adds fmaf((float)v, XS * d, acc) group after group (the prefill
   product in exactly that order; the decode products in the fixed tree documented at kt_tern_gemv), so a token's
   result is the same on every run. */
#ifndef KT_H
#define KT_H

#include <stddef.h>
#include <stdint.h>

#define KT_VERSION 1

#ifdef __cplusplus
extern "C" {
#endif

int kt_version(void);
/* hipSetDevice(device), and the device's address of the library's no-allocation workspace (kt_moe_decode_noalloc).
   gpudrv.py:83-85 (cuCtxSetCurrent) */
int kt_init(int device);
const char* kt_error_string(int rc);

/* ---------------------------------------------------------------- ternary weights
   Device layout "kt2": 2-bit digits + fp16 scale per 128 columns, the same 2.125 bits per weight as the pack.
   kt_tern_weight_bytes: the size of one matrix (rows padded to a multiple of 8), 0 if C % 128 != 0.
   kt_tern_pack: the reference pack of one tensor, unchanged (bcodes [C/4][R]: byte = d0 + 3 d1 + 9 d2 + 27 d3 of
   4 columns, convert.py:49-52, 144-159; dpm [C/128][R] fp16 bits, convert.py:155) -> W (16-byte aligned).
   Replaces layout.repack (layout.py:32-48) and spec.repack / k_tc_pack (spec.py:327-383, tc_hip.cu:31-40). */
size_t kt_tern_weight_bytes(int R, int C);
int kt_tern_pack(const uint8_t* bcodes, const uint16_t* dpm, int R, int C, void* W, void* stream);
/* kt_tern_pack_ptq1: the GGUF tensor itself (type PTQ1_0: per row C / 128 blocks of 28 bytes, qs[24] | qh[2] | fp16
   d, 5 digits a byte; convert.py:33-46 trits_from_raw) -> W, for rows row0 .. row0 + nrows - 1 (row0 % 8 == 0;
   nrows % 8 == 0 unless the range ends at R; raw points at row row0's first block), so a tensor can be streamed
   from a file in row chunks. The same W as kt_tern_pack of convert.py's pack of the tensor. Replaces the offline
   convert + repack path (convert.py:144-159, layout.py:32-48, spec.repack spec.py:327-383). */
int kt_tern_pack_ptq1(const uint8_t* raw, int R, int C, int row0, int nrows, void* W, void* stream);
/* kt_tern_pack_layout: a tensor already in Kindi's load-time GEMV layout (the output of layout.repack, layout.py:32-48,
   as the engine holds it for k_g4 / k_deq_emb3, kindi.cu:525-536): wg4 the repacked bytes [R/16][C/512][4][32][4][4],
   sg4 the scales16 array [R/16][C/512][32][2] (fp16 bits) -> W, the same W as kt_tern_pack of the pack those came
   from. R % 16 == 0 and C % 512 == 0 (layout.py:38-39), else hipErrorInvalidValue. */
int kt_tern_pack_layout(const uint8_t* wg4, const uint16_t* sg4, int R, int C, void* W, void* stream);

/* ---------------------------------------------------------------- activations
   X fp32 [M][ldx] -> XQ int8 [M][ldq] (natural column order, ldq % 16 == 0), XS f32 / XA i32 [M][C/128].
   per_row = 0: the reference's per-128-group scale (k_tc_q8, tc_hip.cu:43-74; tcq128 tc.cu:160-194; k_q8x_T
   chunk.cu:781-802). per_row = 1: one amax per token row (the same formula; XS repeated per group).
   per_row = 2: hp, k_tc_q8 with hp (tc.cu:195-209; KINDI_TC_HP spec.py:63-67): two rows a token, XQ / XS / XA with 2M
   rows. Row 2n is the per-group row of per_row 0; row 2n + 1 quantizes the residual r = fma(-q, amax / 127, x) with
   the fixed amax a2 = amax / 254: q2 = clamp(rne(r (127 / a2)), -127, 127), XS = a2 / 127, XA = sum q2. The decode
   products take such rows with M | KT_HP. Other values: hipErrorInvalidValue. */
#define KT_HP (1 << 30)               /* hp flag, carried in the decode products' M and the producers' HB (tc.cu tc_hp) */
int kt_quant_q8(const float* X, int ldx, int M, int C, int per_row, int8_t* XQ, int ldq, float* XS, int32_t* XA,
                void* stream);

/* ---------------------------------------------------------------- decode products (1 .. 16 tokens a pass)
   Y[n][ldy] = W x_n for tokens n < M. dbg (nullable): the exact group values v, int32 [M][R][C/128].
   Every output row's sum is formed inside one block in a fixed order that depends only on C (never on M or R), so
   a token's result does not depend on how many tokens share the pass. The order: the row's K units are split into
   KS = kt_decode_kslices(C, 0) contiguous slices of whole steps (a step = 8 consecutive units, S steps; KS =
   min(ceil(S / 2), 16); slice k = steps [k S / KS, (k + 1) S / KS)); in a slice, lane c (0..7) chains fmaf over its
   units 8 s + c in increasing order, the 8 lane sums are added by the xor butterfly ((l0 + l1) + (l2 + l3)) +
   ((l4 + l5) + (l6 + l7)), and the slice sums are added left to right. No workspace, no second pass.
   Replaces k_tc_mv{2,4,8} + k_tc_sum (tc_hip.cu:180-199, 236-240, 271-279; spec.py:619-657). */
int kt_decode_kslices(int C, int q8);
/* M | KT_HP (kt_tern_gemv and kt_tern_gemv3): M tokens of two input rows each (kt_quant_q8 per_row 2, or a producer
   with HB | KT_HP); Y row t = the fp32 results of input rows 2t and 2t + 1 added, in that order (tc.cu:405-407).
   Each row's result is the one-row product's, so Y[t] == Y1[2t] + Y1[2t + 1] for the product Y1 of the 2M rows
   without the flag. dbg then has 2M rows. */
int kt_tern_gemv(const void* W, int R, int C, const int8_t* XQ, int ldq, const float* XS, const int32_t* XA, int M,
                 float* Y, int ldy, int32_t* dbg, void* stream);

/* up to three matrices sharing one input (q/k/v, gate/up) in one launch; Y_i is [M][R_i]; R_i <= 0 ends the list.
   Each matrix's outputs are bit-identical to its own kt_tern_gemv. Replaces k_tc_mv3_{2,4,8} (tc_hip.cu:201-234;
   spec.py:659-673). */
int kt_tern_gemv3(const void* W0, int R0, float* Y0, const void* W1, int R1, float* Y1, const void* W2, int R2,
                  float* Y2, int C, const int8_t* XQ, int ldq, const float* XS, const int32_t* XA, int M,
                  void* stream);

/* y[n R + r] = sum over parts p < sp of P[(n sp + p) R + r], in part order. k_tc_sum (tc_hip.cu:271-279). */
int kt_tern_sum(const float* P, float* y, int R, int M, int sp, void* stream);

/* ---------------------------------------------------------------- launch records
   The tuple Kindi's plan holds for each launch, (function, grid, block, kernel arguments), which its HIP path replays
   with hipModuleLaunchKernel (Plan.add tp.py:282-302, Replay.launch spec.py:303-320); it takes the place of the
   function lookup Kindi does on its run-time compiled module (mod.get_function, spec.py:84-93, 202-210).
   kt_record_begin(recs, max): until kt_record_end, every launcher called on this thread validates its arguments as
   always and, instead of launching, appends each of its launches to recs (at most max; the stream argument is not
   used). The kernel, grid and block are the ones the call would have launched for those arguments: a record
   describes that call, with its pointers and sizes, and no other.
   kt_record_end(n): stops recording; *n = the launches the calls made (more than max: hipErrorInvalidValue, the
   first max are filled). A launcher's own validation error is returned by that launcher as always.
   A record: fn is a hipFunction_t; launch it as
     hipModuleLaunchKernel(fn, grid[0], grid[1], grid[2], block[0], block[1], block[2], shmem, stream, args, NULL)
   args[i] points at argument i, stored in the record's own argbuf (at byte off[i]): a record that is copied elsewhere
   must have args rebuilt from off. Records launched in order on one stream give the results of the calls.
   Recording is per thread; calls may not nest. Records of kt_moe_decode_noalloc hold the device address of its
   array. */
#define KT_REC_MAXARGS 24
#define KT_REC_ARGBYTES 512
typedef struct kt_launch {
  void* fn;                           /* hipFunction_t */
  unsigned grid[3], block[3];
  unsigned shmem;                     /* dynamic LDS bytes */
  int nargs;
  void* args[KT_REC_MAXARGS];         /* kernelParams */
  unsigned off[KT_REC_MAXARGS];       /* byte offset of argument i in argbuf */
  uint64_t argbuf[KT_REC_ARGBYTES / 8];
} kt_launch;
int kt_record_begin(kt_launch* recs, int max);
int kt_record_end(int* n);
/* launch records recs[0 .. n) in order, record i on streams[i % nstreams] (1 to 16 streams), with
   hipModuleLaunchKernel: Replay.launch (spec.py:303-320) as one C loop. Launches on different streams carry no
   order between them: a plan whose launches depend on each other (a decode step) takes one stream, as Replay.launch
   replays on one (the null stream); several streams are for records that are independent in turn. */
int kt_replay(const kt_launch* recs, int n, void* const* streams, int nstreams);

/* ---------------------------------------------------------------- prefill product (any M, matrix cores)
   Y and/or Y16 [M][ldy] (fp32 / fp16 bits); dbg as kt_tern_gemv. XA is accepted for the reference's argument list
   and not read (the matrix cores take signed trits). per_row = 0: Y = sum_g fmaf(v, XS[t][g] d[r][g], .) in group
   order (the reference's expression). per_row = 1 (XS from kt_quant_q8 per_row: one scale a token): Y = XS[t][0] *
   sum_g fmaf(v, d[r][g], .) in group order (two VALU operations an element and group instead of three; the same
   bits whichever of the two block shapes R selects, within the 1e-3 tolerance of the reference's expression).
   M ldq, M C / 32 and the packed codes stay below 2^31 bytes. Replaces k_tc_mm2 / k_tc_mm{4,8,16}
   (tc_hip.cu:243-269, chunk.py:273-296) and k_mm_g5q (chunk.cu:858-918, chunk.py:245-271). */
int kt_tern_gemm(const void* W, int R, int C, const int8_t* XQ, int ldq, const float* XS, const int32_t* XA,
                 int per_row, int M, float* Y, uint16_t* Y16, int ldy, int32_t* dbg, void* stream);

/* kt_tern_expand: the signed trits t = d - 1 of W as int8 in natural order, W8 [8 ceil(R/8)][C] (kt_tern_expand_bytes
   bytes, 16-byte aligned; rows past R are padding), the form k_mm_g5q unpacks its tiles into (chunk.cu:836, tq(d) =
   d - 1). Made per call or kept with the weights (4.25 times their bytes).
   kt_tern_gemm8: kt_tern_gemm with per_row = 1 over W8 and W's scales, with the same bits: Y = XS[t][0] *
   sum_g fmaf(v, d[r][g], .) in group order. The product reads both operands into LDS by DMA and unpacks nothing.
   Grids of fewer 128-token x 256-row tiles than 0.7 of the GPU's CUs, and Y / Y16 not 16-byte aligned or ldy not a
   multiple of 8 (the kernel writes 16-byte output rows), run kt_tern_gemm's packed-trit product instead (the same
   bits). M ldq and the W8 bytes stay below 2^31. Replaces k_tc_mm2 (tc_hip.cu:243-269) and k_mm_g5q (chunk.cu:858-918) like
   kt_tern_gemm. */
size_t kt_tern_expand_bytes(int R, int C);
int kt_tern_expand(const void* W, int R, int C, int8_t* W8, void* stream);
int kt_tern_gemm8(const int8_t* W8, const void* W, int R, int C, const int8_t* XQ, int ldq, const float* XS, int M,
                  float* Y, uint16_t* Y16, int ldy, int32_t* dbg, void* stream);

/* ---------------------------------------------------------------- q8_0
   Device layout "kq8": int8 codes + fp16 scale per 32 columns (1.0625 B/w, as GGUF Q8_0).
   kt_q8_pack: GGUF Q8_0 rows (34-byte blocks: fp16 d, 32 int8; dsv41_cpu.c:77-78) -> W. Replaces dg_mat_q8
   (dsv41_gpu.cu:66-88) and the Q8_0 repack of lightning.py.
   kt_q8_quant: X fp32 -> Q int8 [M][ldq] + D f32 [M][ldd] per 32 columns, llama.cpp's CPU rounding
   (d = fp16(amax/127), q = rne(x * 127 / amax); quant_q8 dsv41_cpu.c:251-280, moe_cpu.c:84-112); act = 1 applies
   relu^2 first (lt_quant2, lightning.cu:470). X 16-byte aligned with ldx % 4 == 0, Q 4-byte aligned with
   ldq % 4 == 0.
   kt_q8_gemv: Y = W x for M tokens: per block v = sum w q exact, acc = fmaf((float)v, dw * dx, acc) (lt_mv_q8
   lightning.cu:258-284, k_q8 dsv41_gpu.cu:131-296), summed in kt_tern_gemv's order over 32-column units
   (KS = kt_decode_kslices(C, 1)); dbg int32 [M][R][C/32]. */
size_t kt_q8_weight_bytes(int R, int C);
int kt_q8_pack(const uint8_t* rows, int R, int C, void* W, void* stream);
int kt_q8_quant(const float* X, int ldx, int M, int C, int act, int8_t* Q, int ldq, float* D, int ldd, void* stream);
int kt_q8_gemv(const void* W, int R, int C, const int8_t* Q, int ldq, const float* D, int ldd, int M, float* Y,
               int ldy, int32_t* dbg, void* stream);

/* ---------------------------------------------------------------- MoE
   kt_moe_topk: logits [M][E] -> ids / gw [M][k]: softmax, the k largest (ties to the lower index), weights
   normalized over the chosen k. E <= 1024, k <= 16. A NaN logit ranks below every number (the
   picks stay distinct; its weight is NaN).
   kt_moe_topk_r, kt_moe_route_r, kt_moe_decode_r: the same with the scoring chosen by `score`:
     KT_SCORE_SOFTMAX (0): as above (bias and scale not read);
     KT_SCORE_SIGMOID (1): Kindi's Lightning router (lt_topk / lt_router_topk, lightning.cu:373-468): s_e = 1 / (1 +
     exp(-l_e)), the k largest of s_e + bias[e] (bias [E], device; ties to the lower index), gw_j = s_j / (s_0 + ... +
     s_{k-1}, in pick order) * scale. Exp is expf (the reference's __expf is the fast approximation: the scores'
     last bits may differ from it). Other values, or a NULL bias with KT_SCORE_SIGMOID: hipErrorInvalidValue.
   kt_moe_sort: lt_moe_lists (lightning.cu:1318-1349): cnt / off [E], xrow / where [M k], plus act [E] (experts with
   cnt > 0, ascending) and nact [1]; entries of an expert in ascending t k + j. One block; E <= 1024.
   kt_q8_grouped: per active expert e, Y[p] = W_e x[xrow[p]] for its entries p (xrow NULL: x[p]); Wexp = device
   table of E kq8 buffers (the pointer tables of lt_mv_q2 / lt_mm_*, lightning.cu:154-195, 958-961); M = tokens
   (bounds an expert's list); dbg int32 [entries][R][C/32].
   kt_moe_combine: x[t] += sum_j fmaf(gw[t k + j], yd[where[t k + j]], .) (+ ysh[t]) (lt_moe_combine,
   lightning.cu:1352-1361). */
#define KT_SCORE_SOFTMAX 0
#define KT_SCORE_SIGMOID 1
int kt_moe_topk(const float* logits, int M, int E, int k, int* ids, float* gw, void* stream);
int kt_moe_topk_r(const float* logits, int M, int E, int k, int score, const float* bias, float scale, int* ids,
                  float* gw, void* stream);
int kt_moe_sort(const int* ids, int M, int k, int E, int* cnt, int* off, int* xrow, int* where, int* act, int* nact,
                void* stream);
/* kt_moe_route: kt_moe_topk and kt_moe_sort in one launch (one wave; M k <= 64 entries; the same outputs) — the
   router and list building around lt_router_topk (lightning.cu:414-468) and lt_moe_lists (lightning.cu:1318-1349);
   with x non-NULL, the same launch also writes kt_q8_quant(x, act = 0) into Q / D (H % 32 == 0). */
int kt_moe_route(const float* logits, int M, int E, int k, int* ids, float* gw, int* cnt, int* off, int* xrow,
                 int* where, int* act, int* nact, const float* x, int ldx, int H, int8_t* Q, int ldq, float* D, int ldd,
                 void* stream);
int kt_moe_route_r(const float* logits, int M, int E, int k, int score, const float* bias, float scale, int* ids,
                   float* gw, int* cnt, int* off, int* xrow, int* where, int* act, int* nact, const float* x, int ldx,
                   int H, int8_t* Q, int ldq, float* D, int ldd, void* stream);
int kt_q8_grouped(const void* const* Wexp, int R, int C, int E, const int* cnt, const int* off, const int* act,
                  const int* nact, const int* xrow, int nentries, int M, const int8_t* Q, int ldq, const float* D,
                  int ldd, float* Y, int ldy, int32_t* dbg, void* stream);
int kt_moe_combine(const float* yd, const float* ysh, const int* where, const float* gw, int M, int k, int cols,
                   float* x, void* stream);

/* kt_moe_decode: a q8_0 MoE feed-forward at few tokens (M k <= 64), x [M][ldx] updated in place:
     x[t] += sum_j gw[t][j] down_{e_j}(relu^2(up_{e_j}(x[t])))  (+ ysh[t], stride ldx, nullable)
   with e_j, gw the softmax top-k of logits [M][E] (kt_moe_topk). One token (k <= 8, F <= 4096): two launches; the up
   product routes for itself (every block computes the top-k) and quantizes x in its staging; the down product takes a
   row group of every pick at once, makes relu^2 and the quantization of the intermediate in its staging and adds the
   picks into x in selection order. Otherwise four: kt_moe_route's lists, the grouped up and down products with the
   quantization in their staging, kt_moe_combine. Every intermediate has the bits of the separate launches
   (kt_moe_route + kt_q8_quant + kt_q8_grouped + kt_q8_quant(act 1) + kt_q8_grouped + kt_moe_combine), so x does too.
   Wup / Wdown: device tables of E kq8 buffers ([F x H] and [H x F]); H, F multiples of 32; ldx % 4 == 0, x 16-byte
   aligned. work: a caller buffer of kt_moe_decode_workspace(M, k, E, H, F) bytes (0 = shape not taken), 256-byte
   aligned; its contents need no initialisation, and two calls that overlap in time must not share it. Replaces the
   decode half of Kindi's Lightning MoE layer: lt_router_topk (lightning.cu:414-468), lt_moe_lists (1318-1349),
   lt_quant (70-88), lt_mv_q2 (154-195), lt_quant2 (470), lt_mv_q2_down (197-256) and lt_moe_combine (1352-1361). */
size_t kt_moe_decode_workspace(int M, int k, int E, int H, int F);
int kt_moe_decode(const void* const* Wup, const void* const* Wdown, int E, int H, int F, int k, const float* logits,
                  int M, float* x, int ldx, const float* ysh, void* work, size_t work_bytes, void* stream);
int kt_moe_decode_r(const void* const* Wup, const void* const* Wdown, int E, int H, int F, int k, int score,
                    const float* bias, float scale, const float* logits, int M, float* x, int ldx, const float* ysh,
                    void* work, size_t work_bytes, void* stream);

/* kt_moe_decode_noalloc: kt_moe_decode with its workspace in a device array of the library instead of a caller buffer,
   for callers that cannot allocate device memory (code under graph capture, serving loops that forbid allocation).
   No counterpart in the reference. It allocates nothing and frees nothing; the array (kt_moe_decode_noalloc_max()
   bytes, 4 MiB) is held on every GPU the library runs on until the process ends, and its address on a device is
   resolved by kt_init(device) or by the first call on the device. Shapes whose kt_moe_decode_workspace exceeds it
   return hipErrorInvalidValue. Calls on one GPU share the array: calls that overlap in time on one GPU (other
   streams, other threads) race. The same results as kt_moe_decode (softmax scoring). */
size_t kt_moe_decode_noalloc_max(void);
int kt_moe_decode_noalloc(const void* const* Wup, const void* const* Wdown, int E, int H, int F, int k,
                          const float* logits, int M, float* x, int ldx, const float* ysh, void* stream);

/* ---------------------------------------------------------------- fused input producers
   One launch makes a product's int8 input from the fp32 stream, with the reference's numbers bit for bit:
   kt_rmsfold_q8 replaces k_rmsfold_qT (tcf.cu:370-390; k_rmsfold kindi.cu:350-394): per token row n,
     xf = x + (r_0 + r_1 + ... + r_{nparts-1})   (parts C apart: token n's part p at r + n ldr + p C; 0 <= nparts <= 8)
     xn = (xf * s) * w,  s = 1 / sqrt((float)(S / C) + 1e-6), S the double sum of squares in the reference's order
     xo = fold(sg * xn),  then XQ / XS / XA of xo as kt_quant_q8 (per_row = 0) makes them.
   kt_fold_q8 replaces k_fold_fwht_qT (tcf.cu:410-426): xo = fold(sg * x).
   kt_smfold_q8 replaces k_smfold_qT (tcf.cu:392-408): xo[e] = fold(sg[e] * SiLU(a[s]) * b[s]) with s the grouped-head
     source column of e (rep > 1: e = h + hd (i + rep k) reads h + hd (k + nk i), hd nk rep = C; rep = 1: s = e).
   fold = the unnormalised Walsh-Hadamard transform of each HB-column block times 1/sqrt(HB), HB in {512, 1024,
   4096}. C % HB == 0; rmsfold takes C <= 8192 (one block holds the row for the norm), fold / smfold any width up to
   2^20 (chunks of whole HB blocks). M <= 65535. xw (x + parts, only with nparts > 0), xn and xo are nullable;
   xw, xn and xo may be x itself (with its row stride); they may not overlap x or the parts otherwise.
   HB | KT_HP: the reference's two-row form (hp, ff_q8 tcf.cu:150-205): XQ / XS / XA with 2M rows, row 2n the int8
   row above, row 2n + 1 the residual r = fma(-q, amax / 127, xo) at the fixed scale amax / 32258:
   q2 = clamp(rne(r (32258 / amax)), -127, 127), XS = amax / 32258, XA = sum q2 (0 when amax = 0). */
int kt_rmsfold_q8(const float* x, int ldx, const float* r, int ldr, int nparts, const float* w, const float* sg, int M,
                  int C, int HB, float* xw, int ldxw, float* xn, int ldxn, float* xo, int ldxo, int8_t* XQ, int ldq,
                  float* XS, int32_t* XA, void* stream);
int kt_fold_q8(const float* x, int ldx, const float* sg, int M, int C, int HB, float* xo, int ldxo, int8_t* XQ,
               int ldq, float* XS, int32_t* XA, void* stream);
int kt_smfold_q8(const float* a, int lda, const float* b, int ldb, const float* sg, int hd, int nk, int rep, int M,
                 int C, int HB, float* xo, int ldxo, int8_t* XQ, int ldq, float* XS, int32_t* XA, void* stream);

#ifdef __cplusplus
}
#endif
#endif
