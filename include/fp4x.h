/* fp4x — decode-shaped (M <= 16) quantized GEMV kernels for MI355X (gfx950).
 *
 * C ABI of libfp4x.so.  Every entry point takes raw device pointers, sizes,
 * and the HIP stream to launch on (hipStream_t passed as void*).  Calls are
 * asynchronous on that stream, allocate no device memory, read no device
 * memory from the host, and are capturable into HIP graphs.  They return
 * FP4X_OK (0) or a negative error code; fp4x_last_error() describes the last
 * failure on the calling thread.
 *
 * Bracketed references name the plugin-kernel interface (file:line in the
 * reference tree) each entry point replaces.  Packed layouts are unchanged
 * from the reference:
 *   MXFP8  w u8/e4m3fn [N, K], s u8/e8m0 [N, K/32]
 *   W8 g64 q int8 [N, K], s fp32 (or fp16) [N, K/64]
 *   W6 g32 L u8 [N, K/2] (low nibble = even k), H u8 [N, K/4] (bit pairs of
 *          k%4 = 0, 2, 1, 3), S fp16 [N, K/32]; weight = (lo | hi<<4) - 32
 *   NVFP4  P u8 [N, K/2] (e2m1, low nibble = even k), S e4m3fn [N, K/16], gs fp32
 *   INT2   P u8 [N, K/4] (element j of a 4-group in bit pair (0,2,1,3)[j]),
 *          S fp16 or e4m3fn [N, K/G]; weight = (code - 1.5) * s
 * Activations x are bf16 [M, K] with row stride x_stride elements (16-byte
 * aligned, x_stride % 8 == 0).  Outputs are [M, N] row-major in out_dtype.
 *
 * Split-K (ksplit > 1): `part` is fp32 scratch of fp4x_splitk_sizes()
 * floats and `tickets` int32 scratch of that many counters, zeroed once
 * before first use.  Every call leaves the tickets at zero again.  Calls that
 * share scratch must be ordered (same stream); concurrent calls race.
 */
#ifndef FP4X_H_
#define FP4X_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FP4X_ABI_VERSION 12

enum {
  FP4X_OK = 0,
  FP4X_ERR_ARG = -1,     /* invalid shape, alignment or argument */
  FP4X_ERR_LAUNCH = -2,  /* the HIP runtime rejected a launch */
};

/* dtypes of outputs and scales */
enum { FP4X_DT_BF16 = 0, FP4X_DT_F32 = 1, FP4X_DT_F16 = 2, FP4X_DT_E4M3 = 3 };

/* weight formats (fp4x_layout, fp4x_splitk_sizes, fp4x_dequant_bf16) */
enum {
  FP4X_FMT_MX8 = 0,
  FP4X_FMT_W8_F32 = 1,
  FP4X_FMT_W8_F16 = 2,
  FP4X_FMT_W6 = 3,
  FP4X_FMT_NV4 = 4,
  FP4X_FMT_INT2_F16 = 5,
  FP4X_FMT_INT2_E4M3 = 6,
  FP4X_FMT_BF16 = 7,
};

/* weight-preparation sources and targets (fp4x_quantize, fp4x_absmax) */
enum { FP4X_SRC_F32 = 0, FP4X_SRC_BF16 = 1, FP4X_SRC_MX8 = 2, FP4X_SRC_NV4 = 3 };
enum { FP4X_Q_W8 = 0, FP4X_Q_W6 = 1, FP4X_Q_NV4 = 2, FP4X_Q_INT2 = 3, FP4X_Q_INT2_E4M3 = 4 };

const char* fp4x_last_error(void);
int fp4x_abi_version(void);

/* Lane layout of the rescore kernel (fp4x_refine_mx8) for a row of k_slice
 * weights: lanes per row and 16-byte chunks per lane.  (The GEMV entry
 * points choose their MFMA tiling internally.) */
int fp4x_layout(int fmt, int k_slice, int* lpr, int* cpl);

/* Scratch needed by a split-K call: fp32 slots and int32 tickets. */
int fp4x_splitk_sizes(int fmt, int M, int N, int K, int ksplit, int batch, int64_t* part_floats,
                      int64_t* n_tickets);

/* y = x . bf16(e4m3(w) * 2^(s-127))^T, fp32 accumulate.
 * [mx8_linear -> _run -> _mx8, x/fp4x_kernels.py:65-66, :50-62, :9-29] */
int fp4x_mx8_linear(const void* x, int64_t x_stride, const void* w, const void* s, void* out, int out_dtype,
                    int M, int N, int K, int ksplit, float* part, int* tickets, void* stream);

/* y = x . w^T with bf16 weights w [N, K].
 * [bf16_linear -> _run -> _bg, x/fp4x_kernels.py:69-70, :50-62, :32-47] */
int fp4x_bf16_linear(const void* x, int64_t x_stride, const void* w, void* out, int out_dtype, int M, int N, int K,
                     int ksplit, float* part, int* tickets, void* stream);

/* y = x . bf16(q * s)^T, s fp32 (FP4X_DT_F32, the reference layout) or fp16.
 * [w8_linear -> _run -> _w8, x/fp4x_kernels.py:147-148, :50-62, :116-135] */
int fp4x_w8_linear(const void* x, int64_t x_stride, const void* q, const void* s, int s_dtype, void* out,
                   int out_dtype, int M, int N, int K, int ksplit, float* part, int* tickets, void* stream);

/* fp4x_w8_linear over `layers` independent (x, q, s, out) entries in one
 * launch; *_lstride are the per-layer strides in elements of each tensor.
 * [one w8_linear launch per router gate, x/fp4patch.py:264-272; batching
 * independent layers into one launch is this library's extension] */
int fp4x_w8_linear_layers(const void* x, int64_t x_stride, int64_t x_lstride, const void* q, int64_t q_lstride,
                          const void* s, int s_dtype, int64_t s_lstride, void* out, int out_dtype,
                          int64_t out_lstride, int layers, int M, int N, int K, int ksplit, float* part,
                          int* tickets, void* stream);

/* y = x . bf16(((lo | hi << 4) - 32) * S)^T.
 * [w6_linear -> _run -> _w6, x/fp4x_kernels.py:270-271, :151-176] */
int fp4x_w6_linear(const void* x, int64_t x_stride, const void* L, const void* H, const void* S, void* out,
                   int out_dtype, int M, int N, int K, int ksplit, float* part, int* tickets, void* stream);

/* y = gs * (x . bf16(e2m1(P) * e4m3(S))^T).
 * [nv4_linear -> _nv4, x/fp4x_kernels.py:102-113, :73-99] */
int fp4x_nv4_linear(const void* x, int64_t x_stride, const void* P, const void* S, float gs, void* out,
                    int out_dtype, int M, int N, int K, int ksplit, float* part, int* tickets, void* stream);

/* y = x . bf16((code - 1.5) * S)^T (times rs[n] when rs != NULL), out [M, N].
 * s_fmt = FP4X_DT_F16 or FP4X_DT_E4M3; G = K / S.shape[1].
 * [int2_logits -> _int2_head, x/fp4x_kernels.py:359-364, :304-325] */
int fp4x_int2_logits(const void* x, int64_t x_stride, const void* P, const void* S, int s_fmt, const float* rs,
                     void* out, int out_dtype, int M, int N, int K, int G, void* stream);

/* Top-C of each row of logits [M, V] (dtype FP4X_DT_BF16 or FP4X_DT_F32)
 * under the total order (value descending, then index ascending; -0 equals
 * +0, NaN is largest); idx_out int64 [M, C] lists the selected indices in
 * that order.  C <= min(V, 2048); logits 16-byte aligned with 16-byte aligned
 * rows (stride a multiple of 8 bf16 or 4 fp32 elements).  Rows are read in
 * 16-byte units: each row must be readable up to the next 16-byte boundary
 * past its V elements (the stride gives that to every row but the last; the
 * elements past V are ignored).
 * [torch.topk(coarse, C) in the fast head, x/fp4patch.py:377 (bf16), and
 *  torch.topk(co, dc) in the draft head, x/fp4patch.py:314 (fp32)] */
int fp4x_topk_rows(const void* logits, int dtype, int64_t stride, int M, int V, int C, int64_t* idx_out,
                   void* workspace, int64_t ws_bytes, void* stream);
/* Bytes of device workspace fp4x_topk_rows and fp4x_int2_topk need for M
 * rows of V elements (16-byte aligned, no initial contents required).  Calls
 * that share a workspace must be stream-ordered. */
int64_t fp4x_topk_workspace_size(int M, int V);

/* The coarse stage of the fast head and of the draft head in one call:
 * fp4x_int2_logits into coarse [M, N] (coarse_dtype FP4X_DT_BF16 for the
 * target head, FP4X_DT_F32 for the draft head; 16-byte aligned rows of
 * coarse_stride elements), then fp4x_topk_rows of it into idx_out [M, C],
 * with the top-k's slice maxima written by the coarse kernel's epilogue where
 * it streams.  Results equal the two calls made separately.  set_only != 0:
 * the caller needs the selected set only (both heads scatter exact logits at
 * these indices, so their order does not reach any result); the row's C
 * indices are then the same set in an unspecified order (where the selection
 * can skip the sort it writes them in increasing index order).
 * [int2_logits then torch.topk(coarse, C), x/fp4patch.py:371-377 (bf16);
 *  x/fp4patch.py:313-314 (fp32, the draft head)] */
int fp4x_int2_topk(const void* x, int64_t x_stride, const void* P, const void* S, int s_fmt, const float* rs,
                   void* coarse, int coarse_dtype, int64_t coarse_stride, int M, int N, int K, int G, int C,
                   int64_t* idx_out, int set_only, void* workspace, int64_t ws_bytes, void* stream);

/* fp4x_int2_topk with its workspace (the top-k's slice maxima) in a static
 * device array of the library, fp4x_int2_topk_noalloc_limit() = 1 MiB per
 * device (enough for every M <= 16 and N), instead of a caller's buffer: it
 * allocates nothing.  No counterpart in the reference; it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops).  Requests above the limit return FP4X_ERR_ARG.  Each device's array
 * is found on the first call on that device and kept until the process ends;
 * calls on one device share it, so calls that overlap in time race. */
int fp4x_int2_topk_noalloc(const void* x, int64_t x_stride, const void* P, const void* S, int s_fmt, const float* rs,
                           void* coarse, int coarse_dtype, int64_t coarse_stride, int M, int N, int K, int G, int C,
                           int64_t* idx_out, int set_only, void* stream);
int64_t fp4x_int2_topk_noalloc_limit(void);

/* In place: out[m, idx[m, c]] = cast(sum_k float(e4m3(w)*2^(s-127)) * float(x[m, k])).
 * out is [M, V] in out_dtype, x bf16 [M, K] contiguous, idx int64 [M, C].
 * [refine_mx8_ -> _refine_mx8, x/fp4x_kernels.py:384-388, :367-381] */
int fp4x_refine_mx8(void* out, int out_dtype, int64_t out_stride, const void* x, const int64_t* idx, int M, int C,
                    const void* w, const void* s, int K, int V, void* stream);

/* Exact NVFP4 logits of candidate rows: out [M, C] fp32,
 * out[m, c] = (sum_k float(bf16(e2m1(wp) * e4m3(s))) * float(x[m, k])) * gs,
 * in the rescore kernel's specified fma order; NaN where idx[m, c] is outside
 * [0, V).  wp [V, K/2] (low nibble = even k), s [V, K/16] e4m3, K % 32 == 0.
 * [refine_nv4 -> _refine_nv4, x/fp4x_kernels.py:410-415, :391-407; the draft
 *  head, x/fp4patch.py:316] */
int fp4x_refine_nv4(float* out, const void* x, const int64_t* idx, int M, int C, const void* wp, const void* s, float gs,
                    int K, int V, void* stream);

/* Draft logits out [M, vocab] bf16 (row stride out_stride): -inf everywhere
 * except out[m, ids[cand[m, c]]] = bf16(vals[m, c] * *inv_t) (bf16(vals[m, c])
 * when inv_t is NULL).  vals fp32 [M, C], cand int64 [M, C] indexing ids,
 * ids int64 [n_ids] column numbers; entries whose cand or ids value is out of
 * range are not written.  Every element of out is written, so out need not be
 * initialised.  inv_t is a device pointer (read on the device: graph-safe).
 * [the draft head's full(-inf) + scatter_, x/fp4patch.py:316-320] */
int fp4x_scatter_draft(void* out, int64_t out_stride, const float* vals, const int64_t* cand, const int64_t* ids,
                       int64_t n_ids, const float* inv_t, int M, int C, int64_t vocab, void* stream);

/* Draft logits out [M, vocab] bf16 (row stride out_stride) straight from the
 * candidates: fp4x_refine_nv4 over the rows cand[m, c] of the NVFP4 matrix
 * (wp [n_ids, K/2], s [n_ids, K/16], gs) followed by fp4x_scatter_draft of
 * its sums to columns ids[cand[m, c]], in one launch and bit for bit:
 * out[m, ids[cand[m, c]]] = bf16((sum * gs) * *inv_t) (bf16(sum * gs) when
 * inv_t is NULL), -inf elsewhere.  The matrix rows and ids are the subset's,
 * one per row; a cand value outside [0, n_ids) or an ids value outside
 * [0, vocab) is not written.  C <= 2048, K % 32 == 0, n_ids > 0 (when M and
 * C are); x bf16 [M, K] and wp
 * 16-byte aligned.  [the draft head's rescore + full(-inf) + scatter_,
 * x/fp4x_kernels.py:391-416 and x/fp4patch.py:316-320] */
int fp4x_draft_nv4(void* out, int64_t out_stride, const void* x, const int64_t* cand, const int64_t* ids,
                   int64_t n_ids, const void* wp, const void* s, float gs, const float* inv_t, int M, int C, int K,
                   int64_t vocab, void* stream);

/* Weight preparation: quantize an [N, K] matrix (K % 64 == 0) group by group.
 * Source src: FP4X_SRC_F32 / _BF16 (src_a rows, contiguous), _MX8 (src_a
 * e4m3fn [N, K], src_b e8m0 [N, K/32]) or _NV4 (src_a e2m1 pairs [N, K/2],
 * src_b e4m3fn [N, K/16], src_gs), packed rows decoded exactly as by
 * mx8_dequant and dequant_nv4.  Target dst:
 *   FP4X_Q_W8   out0 int8 q [N, K], out1 fp32 s [N, K/64]
 *   FP4X_Q_W6   out0 L [N, K/2], out1 H [N, K/4], out2 fp16 S [N, K/32]; qmax 1..31
 *   FP4X_Q_NV4  out0 P [N, K/2], out1 e4m3fn S [N, K/16]; dst_gs the global scale
 *   FP4X_Q_INT2 out0 P [N, K/4], out1 fp16 S [N, K/G]; G = 16, 32 or 64
 *   FP4X_Q_INT2_E4M3 out0 P [N, K/4], out1 e4m3fn S [N, K/G], out2 fp32 row
 *               scales [N]; G = 16, 32 or 64 (scale_fmt "e4m3")
 * Results equal the reference's torch quantizers evaluated in fp32 with IEEE
 * division.  16-byte aligned sources and out0.
 * [quantize_w8 :138-144, quantize_w6 :179-202 (clip_search = 0), quantize_nv4
 *  :277-300, quantize_int2 :330-351 (fp16 or e4m3 scales); the weight preparation of
 *  x/fp4patch.py:61-83, :179-182, :211-214, :357-359] */
int fp4x_quantize(int src, const void* src_a, const void* src_b, float src_gs, int64_t N, int K, int dst, int G,
                  int qmax, float dst_gs, void* out0, void* out1, void* out2, void* stream);
/* W6 g32 with the clip search: per group, the scale among s = max(fp16(amax /
 * qmax), 6.2e-5) and max(fp16(s * c_i), 6.2e-5), c_i = torch.linspace(0.70,
 * 0.98, clip_search) in fp32, with the strictly smallest squared error (fp32,
 * summed in the order of torch's CPU sum over the group's 32 squares); then
 * the codes and planes of FP4X_Q_W6.  Sources as fp4x_quantize; qmax 1..31,
 * clip_search 0..64 (0: the plain W6 target).  L [N, K/2] 16-byte aligned,
 * H [N, K/4] 8-byte aligned, S fp16 [N, K/32].
 * [quantize_w6 with clip_search, x/fp4x_kernels.py:179-202; the dense layer
 *  preparation under FP4X_DENSE_CLIP, x/fp4patch.py:66-83] */
int fp4x_quantize_w6_clip(int src, const void* src_a, const void* src_b, float src_gs, int64_t N, int K, int qmax,
                          int clip_search, void* L, void* H, void* S, void* stream);
/* max |w| of a source matrix (as fp4x_quantize reads it) into *out, a device
 * float the caller zeroes first.  [quantize_nv4's global amax, x/fp4x_kernels.py:284-287] */
int fp4x_absmax(int src, const void* src_a, const void* src_b, float src_gs, int64_t N, int K, float* out,
                void* stream);

/* Mixer down projection: split-K W8 GEMV whose last workgroup per row tile
 * writes di = bf16(sum) [M, N] and bot = bf16(sc * sigmoid(sc)) [M, lr] with
 * sc = bf16(di / hc), then re-arms its ticket.
 * [HCFused.down -> _hc_down, x/fp4x_kernels.py:503-510, :438-467] */
int fp4x_hc_down(const void* x, int64_t x_stride, const void* q, const void* s, int s_dtype, void* di, void* bot,
                 int M, int N, int K, int lr, int hc, int ksplit, float* part, int* tickets, void* stream);

/* Mixer up projection over stream-interleaved rows (tile of hc*bj rows holds
 * rows s*H + j*bj + t), with the gate/stream-mean epilogue:
 * out[m, j] = bf16(sum_s bf16(nrm[m, s*H + j] * bf16(sigmoid(bf16(acc)))) / hc).
 * [HCFused.up -> _hc_up, x/fp4x_kernels.py:519-526, :470-493] */
int fp4x_hc_up(const void* bot, int64_t bot_stride, const void* qi, const void* si, int s_dtype, const void* nrm,
               int64_t nrm_stride, void* out, int M, int K, int H, int hc, int bj, void* stream);

/* Whole mixer, fp4x_hc_down followed by fp4x_hc_up on its bottleneck
 * (bot [M, lr] contiguous, up K = lr, one scale dtype for both), with results
 * bit-identical to those two calls.  When both halves take their planned
 * decompositions it runs as one launch (the up weights stream while the down
 * projection runs); otherwise it makes the two calls.  tickets: n_tickets
 * int32, zero before the first call and never touched by the caller
 * afterwards.  The single launch keeps one tile ticket per 128-byte line,
 * ticket t at 32 t, and at S = (n_tickets - 32 * (CUs + 1)) rounded down to
 * a multiple of 32 an unused word (S), a status word (S + 1) and one
 * 128-byte line per workgroup slot (its generation flag, its ack word and
 * its call count), so it needs S >= 32 * ceil(N / 16); with fewer it makes
 * the two calls.  (S depends on the buffer alone: calls of any shape on one
 * buffer agree on it.)  The launch has one workgroup per CU; every call
 * counts in every slot, so all slots agree on the call's count, which tags
 * the down partials.  part: zero before the first call; the single launch
 * keeps the down partials of each tile on one XCD as 64-bit (partial, tag)
 * pairs after the two calls' slots (8-byte aligned part; 3 * ceil(N / 16) *
 * 16 * M * (parts per tile) + 2 floats, else device-coherent partials).  A
 * workgroup whose flag wait gives up (only
 * possible when other work holds the GPU's CUs for about a second) writes NaN
 * to its outputs and sets bit 0 of the status word; a down tile whose closer
 * gives up waiting for a part's pairs (a part placed on another XCD, or held
 * off the CUs as long) writes NaN and sets bit 1; the next call is not
 * affected.
 * FP4X_HC_MIX=0 forces the two calls, FP4X_HC_XCD=0 device-coherent
 * partials.
 * [HCFused.down then HCFused.up as the plugin's fused mixer calls them,
 *  x/fp4patch.py:217-218 (_mix_fused); x/fp4x_kernels.py:503-526] */
int fp4x_hc_mix(const void* x, int64_t x_stride, const void* q, const void* s, int s_dtype, void* di, void* bot,
                int M, int N, int K, int lr, int hc, int ksplit, float* part, int* tickets, int n_tickets,
                const void* qi, const void* si, const void* nrm, int64_t nrm_stride, void* out, int H, int bj,
                void* stream);

/* Unfused mixer epilogues (the b12x run_scaled_silu / run_gate_mean ops the
 * plugin calls, x/fp4patch.py:238-246, at the rounding points of
 * x/fp4x_kernels.py:461-464 and :486-493).
 * scaled_silu: bot[m, n] = bf16(sc * sigmoid(sc)), sc = bf16(d[m, n] / hc), n < lr.
 * gate_mean:   out[m, j] as in fp4x_hc_up, from bf16 gate logits g [M, hc*H]. */
int fp4x_hc_scaled_silu(const void* d, int64_t d_stride, void* bot, int M, int lr, int hc, void* stream);
int fp4x_hc_gate_mean(const void* nrm, int64_t nrm_stride, const void* g, int64_t g_stride, void* out, int M, int H,
                      int hc, void* stream);

/* bf16 operand of each weight as the GEMV kernels decode it, out bf16 [N, K].
 * w0/w1/s are the format's planes (w1 only for W6).
 * [the in-kernel dequant of _mx8/_w8/_w6/_nv4/_int2_head, x/fp4x_kernels.py:19-23,
 *  :126-129, :161-170, :84-92, :317-322] */
int fp4x_dequant_bf16(int fmt, const void* w0, const void* w1, const void* s, int N, int K, int G, void* out,
                      void* stream);

/* fp32 MXFP8 dequant, out [N, K].  [mx8_dequant, x/fp4x_kernels.py:261-267] */
int fp4x_mx8_dequant(const void* w, const void* s, int N, int K, float* out, void* stream);

/* A plain coalesced read of `bytes` (a multiple of 16, src 16-byte aligned)
 * with `unroll` (2, 4, 8 or 16) 16-byte loads in flight per thread over
 * wgs_per_cu (1..32) workgroups of 256 threads per CU; *sink is written only
 * if the data fold to one particular word.  No counterpart in the reference:
 * the benchmark's measured ceiling of a one-shot read of a GEMV's bytes. */
int fp4x_read_ceiling(const void* src, int64_t bytes, int unroll, int wgs_per_cu, uint32_t* sink, void* stream);

/* Launch `wgs` one-wave workgroups on `stream` that each hold a CU for
 * `microseconds` of wall-clock time (at most 100 ms) and then end; each
 * takes lds_kb KB of LDS (up to 160, a whole CU's), which keeps workgroups
 * that need LDS off its CU meanwhile.  No counterpart in the reference: a
 * test utility, with which the mixer's tests make its workgroups start late,
 * as when another kernel holds part of the GPU. */
int fp4x_hold_cus(int wgs, int64_t microseconds, int lds_kb, uint32_t* sink, void* stream);

/* Re-read the path switches from the environment (they are read once, when
 * first needed, never per launch): FP4X_W8_STREAM, FP4X_INT2_STREAM,
 * FP4X_NV4_STREAM, FP4X_W6_STREAM, FP4X_MX8_STREAM and FP4X_HC_MIX ("0"
 * selects the MFMA core or the two-call mixer), FP4X_HC_XCD ("0": the
 * single-launch mixer's down partials device-coherent rather than in one
 * XCD's L2), FP4X_ROWS, FP4X_WAVES_PER_CU, FP4X_HC_SPIN_LIMIT.  Not
 * thread-safe against concurrent launches.  No counterpart in the reference
 * (its Triton launches take no such switches). */
int fp4x_reload_env(void);

#ifdef __cplusplus
}
#endif

#endif /* FP4X_H_ */
