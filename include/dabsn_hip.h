/*
 * dabsn_hip.h -- C ABI of the MI355X (gfx950) DABSN hot-path library.
 *
 * Every entry point takes raw device pointers, sizes and a hipStream_t, enqueues its
 * kernels on that stream (no host synchronisation inside) and returns a status code:
 * 0 on success, negative on error (dabsn_hip_last_error() describes it). Tensors are
 * dense row-major. `dtype` selects the activation storage type: 0 = fp32, 1 = bf16
 * (raw 16-bit storage); per-unit parameters, carried states and reductions are fp32.
 *
 * Each entry point names the reference interface it replaces (paths relative to the
 * BleedingXiko/dabsn source tree).
 */
#ifndef DABSN_HIP_H_
#define DABSN_HIP_H_

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#define DABSN_HIP_ABI_VERSION 18

/* Status codes returned by every entry point. */
#define DABSN_OK 0
#define DABSN_ERR_HIP (-1)         /* a HIP runtime call failed */
#define DABSN_ERR_ARG (-2)         /* invalid argument (shape, pointer, workspace size) */
#define DABSN_ERR_UNSUPPORTED (-3) /* configuration this build or device cannot run */

#ifdef __cplusplus
extern "C" {
#endif

/* ---- library ----------------------------------------------------------------- */
int dabsn_hip_abi_version(void);
const char* dabsn_hip_last_error(void);
/* Zero `bytes` (multiple of 4) of device memory with a fill kernel (graph-safe). */
int dabsn_hip_zero(void* ptr, size_t bytes, hipStream_t stream);

/* ---- core recurrence ------------------------------------------------------------
 * Replaces the device kernels of the registered op dabsn::core_scan_batched
 * (src/dabsn/kernels/batched_runtime.py:1507-1586; CPU kernel cpu.py:777-882 ->
 * cpu_runtime.cpp:672-837) and its reverse recurrence (batched_runtime.py:299-466,
 * 1333-1504), which the reference only has as a Python per-step loop.
 *
 * Parameter table: vec[16] are [H] fp32 vectors in op-input order 4..19 (beta, log_kappa,
 * logit_recover, k_s, k_y, k_b, k_n, k_bias, r_s, r_y, r_b, r_n, r_bias, logit_c_decay,
 * k_c, r_c); scal[3] point at fp32 scalars (logit_alpha, log_lambda, logit_c_suppress).
 * The workspace's first 4 bytes hold an error word (non-zero = a step barrier timed out);
 * the caller may read it after the stream completes. */
typedef struct dabsn_core_params {
  const float* vec[16];
  const float* scal[3];
} dabsn_core_params;

size_t dabsn_hip_core_scan_workspace_bytes(int dtype, int64_t B, int64_t H, int backward);

/* Number of batch groups and of workgroups: sizes of part_vec ([nbg][16][H]) and
 * part_scal ([nwg][3]) in the backward. */
int dabsn_hip_core_scan_layout(int dtype, int64_t B, int64_t H, int64_t* nbg, int64_t* nwg);

/* Number of cooperative launches a scan of (dtype, B, T, H) makes on the current device:
 * 1 when every batch group is resident in one launch; more when the batch runs as
 * consecutive launches over slabs of batch groups; 0 for T == 0 and for the forward of
 * T == 1, which runs the one-step path without a cooperative launch. */
int dabsn_hip_core_scan_launches(int dtype, int64_t B, int64_t T, int64_t H, int backward,
                                 int64_t* launches);

/* Launch configuration chosen for (dtype, B, H): channels per workgroup, MFMA k-steps per
 * wave and waves per workgroup (names the kernel instance in profiler output). */
int dabsn_hip_core_scan_config(int dtype, int64_t B, int64_t H, int* ch, int* ksteps, int* waves);

/* Forward. Wx, Wgx [B,T,H]; GA = [Ug; A] as [2H,H]; b0, e0, c0 [B,H] fp32.
 * Outputs: U [B,T,2H] (y, next budget), nov, plast, expr, write, energy (pre-update),
 * sat (post-update), gate [B,T,H]; final state bF, eF, cF [B,H] fp32.
 * bf16 with H >= 1024 moves rows as 16-byte chunks: H must be a multiple of 16 and Wx, Wgx
 * and the tape pointers 16-byte aligned (DABSN_ERR_ARG otherwise); the backward asks
 * the same of its tapes, grads and outputs. Any B: batch groups that do not fit on the
 * device at once run as consecutive launches on the same stream. */
int dabsn_hip_core_scan_fwd(int dtype, int64_t B, int64_t T, int64_t H, const void* Wx,
                            const void* Wgx, const void* GA, const dabsn_core_params* params,
                            const float* b0, const float* e0, const float* c0, void* U, void* nov,
                            void* plast, void* expr, void* write, void* energy, void* sat,
                            void* gate, float* bF, float* eF, float* cF, void* workspace,
                            size_t workspace_bytes, hipStream_t stream);

/* Backward. GAT = [Ug; A]^T as [H,2H]. Saved tapes from the forward; upstream grads gU
 * [B,T,2H], gNov, gP, gAy, gW, gE, gC [B,T,H] and gbF, geF, gcF [B,H] (any may be NULL =
 * zeros). Outputs: gWx, gWgx (= d gate pre-activation), day (= d expression) [B,T,H];
 * per-unit parameter partials part_vec [nbg][16][H]; scalar partials part_scal [nwg][3];
 * initial-state grads gb0, ge0, gc0 [B,H]. grad [Ug; A] = [gWgx; day]^T y is a plain GEMM
 * left to the caller. */
int dabsn_hip_core_scan_bwd(int dtype, int64_t B, int64_t T, int64_t H, const void* GAT,
                            const dabsn_core_params* params, const float* b0, const float* c0,
                            const void* U, const void* plast, const void* expr, const void* energy,
                            const void* sat, const void* gate, const void* gU, const void* gNov,
                            const void* gP, const void* gAy, const void* gW, const void* gE,
                            const void* gC, const float* gbF, const float* geF, const float* gcF,
                            void* gWx, void* gWgx, void* day, float* part_vec, float* part_scal,
                            float* gb0, float* ge0, float* gc0, void* workspace,
                            size_t workspace_bytes, hipStream_t stream);

/* Call descriptors: the arguments of dabsn_hip_core_scan_fwd / _bwd, plus `ldt`, the
 * number of time steps between consecutive batch rows of every [B, *, .] tensor of the
 * call (0 = T, i.e. dense). With ldt > T the call scans a time window [t0, t0 + T) of
 * longer sequences in place: every pointer is offset to step t0 and rows are ldt apart. */
typedef struct dabsn_core_fwd_call {
  int dtype;
  int64_t B, T, H, ldt;
  int64_t ldx; /* elements between consecutive time steps of Wx and Wgx: 0 = H (dense);
                  2H reads the two halves of one [B, T, 2H] projection (core.py:281-282 as
                  one GEMM over [W; Wg]). Above H it must be a multiple of 8. */
  const void *Wx, *Wgx, *GA;
  const dabsn_core_params* params;
  const float *b0, *e0, *c0;
  void *U, *nov, *plast, *expr, *write, *energy, *sat, *gate;
  float *bF, *eF, *cF;
  void* workspace;
  size_t workspace_bytes;
  int state_dtype; /* type of b0, e0, c0 and of bF, eF, cF: 0 = fp32, 1 = bf16 (the state
                      carried in the activation dtype, as the reference's streaming memory
                      does, src/dabsn/memory.py:228-232; the final state rounded to nearest
                      even). The pointers keep their float* type either way. */
  int coresident_cus; /* 0: cooperative launches (the runtime guarantees that every
                         workgroup is resident; nothing else runs beside them). > 0: plain
                         launches, for a stream restricted to that many CUs (e.g. one of
                         dabsn_hip_stream_pair's) on which nothing else runs during the scan:
                         the caller guarantees residency and work on the other CUs overlaps
                         the scan. Barrier waits stay bounded either way. */
} dabsn_core_fwd_call;

typedef struct dabsn_core_bwd_call {
  int dtype;
  int64_t B, T, H, ldt;
  const void* GAT;
  const dabsn_core_params* params;
  const float *b0, *c0;
  const void *U, *plast, *expr, *energy, *sat, *gate;
  const void *gU, *gNov, *gP, *gAy, *gW, *gE, *gC;
  const float *gbF, *geF, *gcF;
  void *gWx, *gWgx, *day;
  float *part_vec, *part_scal, *gb0, *ge0, *gc0;
  void* workspace;
  size_t workspace_bytes;
  int coresident_cus; /* as in dabsn_core_fwd_call */
} dabsn_core_bwd_call;

int dabsn_hip_core_scan_fwd_call(const dabsn_core_fwd_call* fwd, hipStream_t stream);
int dabsn_hip_core_scan_bwd_call(const dabsn_core_bwd_call* bwd, hipStream_t stream);

/* Two streams on complementary halves of the device's CUs (hipExtStreamCreateWithCUMask;
 * on MI355X each gets 16 CUs of every XCD), for overlapping the persistent core scan
 * (plain launches with coresident_cus = *cus_a) with other work. No reference
 * counterpart: the reference's scan is a sequence of per-step launches. *cus_a and *cus_b
 * receive the CU counts of the two masks. Release each with dabsn_hip_stream_destroy. */
int dabsn_hip_stream_pair(hipStream_t* a, hipStream_t* b, int* cus_a, int* cus_b);

/* Waits for the work on a stream made by dabsn_hip_stream_pair and destroys it. No
 * reference counterpart (the reference makes no streams of its own); the Python binding
 * calls it at interpreter exit, before the runtime's own teardown. */
int dabsn_hip_stream_destroy(hipStream_t stream);

/* ---- linear recurrence -----------------------------------------------------------
 * Replaces dabsn::linear_recurrence / dabsn::_linrec_backward
 * (src/dabsn/kernels/long.py:392-437; CPU cpu_runtime.cpp:92-143).
 * y_t = a_t * y_{t-1} + g_t over [B,T,H], y_{-1} = y0 [B,H] (same dtype as a).
 * Backward workspace: dabsn_hip_linrec_workspace_bytes() bytes. */
int dabsn_hip_linrec_fwd(int dtype, int64_t B, int64_t T, int64_t H, const void* a, const void* g,
                         const void* y0, void* y, hipStream_t stream);
size_t dabsn_hip_linrec_workspace_bytes(int dtype, int64_t B, int64_t T, int64_t H);
int dabsn_hip_linrec_bwd(int dtype, int64_t B, int64_t T, int64_t H, const void* a, const void* g,
                         const void* y0, const void* gy, void* da, void* dg, void* dy0,
                         void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ---- recurrent long memory ---------------------------------------------------------
 * Fused form of the three recurrences of src/dabsn/kernels/long.py:492-579 (loop form
 * read.py:625-636). logits[4] point at fp32 scalars (logit_expect_retain,
 * logit_retention_decay, logit_retain, logit_retention_strength). State L0/E0/R0 [B,H]
 * fp32 in, LF/EF/RF out. Both directions are chunked over time (chunks of DABSN_LONG_CKPT
 * steps) and need dabsn_hip_long_workspace_bytes() bytes of workspace. `ckpt` (may be NULL)
 * receives the checkpoint the backward replays each chunk from: the fp32 states entering
 * every chunk, [B][ceil(T / DABSN_LONG_CKPT)][3][H] = (L, E, R). `ldx`: elements between
 * the batch rows of w and p (0: T H, contiguous; otherwise >= T H, e.g. a time window of
 * longer [B, T', H] tapes read in place); out and every other tensor are contiguous. */
#define DABSN_LONG_CKPT 32
size_t dabsn_hip_long_workspace_bytes(int64_t B, int64_t T, int64_t H, int backward);
int dabsn_hip_long_fwd(int dtype, int64_t B, int64_t T, int64_t H, int64_t ldx, const void* w,
                       const void* p, const float* const* logits, const float* L0,
                       const float* E0, const float* R0, void* out, float* LF, float* EF,
                       float* RF, float* ckpt, void* workspace, size_t workspace_bytes,
                       hipStream_t stream);
/* Backward: gout [B,T,H] (contiguous), gLF/gEF/gRF (may be NULL), the forward's `ckpt`, w
 * and p with the forward's `ldx`. Outputs gw, gp [B,T,H] with batch stride `ldo` (0: T H;
 * e.g. time windows of full-length gradient buffers written in place), gL0, gE0, gR0 [B,H],
 * and part_logit [nblocks][4] with nblocks = dabsn_hip_long_partials(B, T, H): per-block
 * partial sums of the gradient w.r.t. the four logits. gw_accumulate != 0: gw receives
 * gw + (the gradient rounded to dtype), summed in fp32 and rounded once -- an add into an
 * existing gradient buffer. */
int64_t dabsn_hip_long_partials(int64_t B, int64_t T, int64_t H);
int dabsn_hip_long_bwd(int dtype, int64_t B, int64_t T, int64_t H, int64_t ldx, const void* w,
                       const void* p, const float* const* logits, const float* ckpt,
                       const void* gout, const float* gLF, const float* gEF, const float* gRF,
                       void* gw, void* gp, int64_t ldo, int gw_accumulate, float* gL0,
                       float* gE0, float* gR0, float* part_logit, void* workspace,
                       size_t workspace_bytes, hipStream_t stream);

/* ---- read glue ----------------------------------------------------------------------
 * Per-position statistics of the read (src/dabsn/read.py:58-72, 154-183): stats[B,T,6] =
 * (mean energy, mean saturation, mean novelty, mean plasticity, |expression|, |write|). */
int dabsn_hip_tape_stats(int dtype, int64_t B, int64_t T, int64_t H, const void* nov,
                         const void* plast, const void* energy, const void* sat, const void* expr,
                         const void* write, float* stats, hipStream_t stream);
/* Backward of tape_stats' means: each of gnov, gplast, genergy, gsat [B,T,H] (NULL to skip)
 * receives its mean's gradient / H, written (accumulate = 0) or added (accumulate = 1).
 * The norms' gradients belong to the normalisation and gather backward passes. */
int dabsn_hip_tape_stats_bwd(int dtype, int64_t B, int64_t T, int64_t H, const float* gstats,
                             int accumulate, void* gnov, void* gplast, void* genergy, void* gsat,
                             hipStream_t stream);
/* The two above on a time window [t0, t0 + T) of longer sequences, in place: the tape (and
 * tape-gradient) pointers point at step t0 of batch row 0 with batch rows ldt steps apart,
 * the statistics rows lds rows apart (no copies of the window). */
int dabsn_hip_tape_stats_window(int dtype, int64_t B, int64_t T, int64_t H, int64_t ldt,
                                const void* nov, const void* plast, const void* energy,
                                const void* sat, const void* expr, const void* write,
                                float* stats, int64_t lds, hipStream_t stream);
int dabsn_hip_tape_stats_bwd_window(int dtype, int64_t B, int64_t T, int64_t H, int64_t ldt,
                                    const float* gstats, int64_t lds, int accumulate, void* gnov,
                                    void* gplast, void* genergy, void* gsat, hipStream_t stream);
/* Read output (src/dabsn/read.py:435-438, 821-823): out = proj + gain * long over n
 * elements, as the reference's two tensor operations under type promotion: the product in
 * prod_dtype (the promotion of gain and long), the sum in out_dtype (the promotion of proj
 * and the product); no fused multiply-add. gain points at one fp32 value. */
int dabsn_hip_read_output(int proj_dtype, int long_dtype, int prod_dtype, int out_dtype,
                          int64_t n, const void* proj, const void* lng, const float* gain,
                          void* out, hipStream_t stream);
/* Its backward: gproj = gout in proj_dtype; glong = (gout in prod_dtype) * gain in
 * prod_dtype, stored in long_dtype; ggain (one fp32 value) = the sum of (gout in prod_dtype)
 * * long, reduced in a fixed order through `partials`, partial_count >=
 * dabsn_hip_read_output_partials(n) floats of scratch. */
size_t dabsn_hip_read_output_partials(int64_t n);
int dabsn_hip_read_output_bwd(int out_dtype, int proj_dtype, int long_dtype, int prod_dtype,
                              int64_t n, const void* gout, const void* lng, const float* gain,
                              void* gproj, void* glong, float* ggain, float* partials,
                              size_t partial_count, hipStream_t stream);
/* The two above on a window of rows: `rows` segments of row_len elements, each tensor's
 * segments its own ld_* elements apart (a time window [t0, t1) of a [B, T, H] tensor:
 * rows = B, row_len = (t1 - t0) H, ld = T H, pointer at step t0 of batch row 0; a
 * contiguous [B, t1 - t0, H] block: ld = row_len). The backward's partial_count >=
 * dabsn_hip_read_output_partials(rows * row_len); ggain receives the window's share of the
 * gain gradient. No reference counterpart: they let a time-chunked read form its output and
 * gradient window by window. */
int dabsn_hip_read_output_window(int proj_dtype, int long_dtype, int prod_dtype, int out_dtype,
                                 int64_t rows, int64_t row_len, int64_t ld_proj,
                                 int64_t ld_long, int64_t ld_out, const void* proj,
                                 const void* lng, const float* gain, void* out,
                                 hipStream_t stream);
int dabsn_hip_read_output_bwd_window(int out_dtype, int proj_dtype, int long_dtype,
                                     int prod_dtype, int64_t rows, int64_t row_len,
                                     int64_t ld_gout, int64_t ld_long, int64_t ld_gproj,
                                     int64_t ld_glong, const void* gout, const void* lng,
                                     const float* gain, void* gproj, void* glong, float* ggain,
                                     float* partials, size_t partial_count, hipStream_t stream);
/* Row normalisation q = x / max(|x|, 1e-12) given norms [B*T] (F.normalize, read.py:154). */
int dabsn_hip_normalize_rows(int dtype, int64_t rows, int64_t H, const void* x, const float* norms,
                             void* q, hipStream_t stream);
/* Backward: gx += (gq - q (q . gq)) / max(|x|, eps). */
int dabsn_hip_normalize_rows_bwd(int dtype, int64_t rows, int64_t H, const void* q,
                                 const float* norms, const void* gq, void* gx, hipStream_t stream);

/* Key bias, admission and cocktail from rows of tape statistics (read.py:58-72, 155-180,
 * 680-700): stats rows of 6 fp32 (mean energy, saturation, novelty, plasticity, query
 * norm, write norm), row n of batch b at stats + b * ld + 6 n; params = 8 fp32 device
 * scalars (p_gain, novelty_gain, null_bias, adm_p_gain, adm_novelty_gain,
 * adm_saturation_gain, adm_energy_gain, adm_bias); outputs key_bias, admission [B, N]
 * (either may be NULL) and cocktail [B, N, 4] = normalize(means) (16-byte aligned).
 * `mode` gives the dtype the reference evaluates the expressions in: 0 = fp32; bit 0 =
 * bf16 tapes (the means and the tape-dtype intermediates are rounded to bf16); bit 1 (with
 * bit 0) = bf16 gains as well (every product and sum rounded to bf16). */
int dabsn_hip_means_glue(int64_t B, int64_t N, int64_t ld, const float* stats, int64_t hidden,
                         const float* const* params, int mode, float* key_bias, float* admission,
                         float* cocktail, hipStream_t stream);
/* The same expressions for the admitted slots of a read (replaces read.py:241-256's
 * torch.gather of the key bias, admission and cocktail by slot): for slot j of row b,
 * the glue of bank row idx[b][j] (clamped into [0, L)) of stats (rows of batch b at stats +
 * b * ld). Outputs [B, N] and [B, N, 4] (16-byte aligned). */
int dabsn_hip_glue_slots(int64_t B, int64_t N, int64_t L, int64_t ld, const float* stats,
                         const int64_t* idx, int64_t hidden, const float* const* params, int mode,
                         float* key_bias, float* admission, float* cocktail, hipStream_t stream);
/* Backward of dabsn_hip_glue_slots: the four mean gradients of slot j's bank row are written
 * to gstats + b * ldg + 6 idx[b][j] (columns 0..3; the slots of a row are distinct
 * positions, every other row is left as it is), and gparams[8] receives the eight
 * parameter gradients, summed in a fixed order through `partial`
 * (dabsn_hip_glue_slots_partials(B, N) bytes). Evaluated in fp32 from the forward's means
 * and intermediates, rounded as the forward rounds them. */
size_t dabsn_hip_glue_slots_partials(int64_t B, int64_t N);
int dabsn_hip_glue_slots_bwd(int64_t B, int64_t N, int64_t L, int64_t ld, const float* stats,
                             const int64_t* idx, int64_t hidden, const float* const* params,
                             int mode, const float* gkey_bias, const float* gadmission,
                             const float* gcocktail, float* gstats, int64_t ldg, float* partial,
                             float* gparams, hipStream_t stream);
/* Backward of the cocktail of rows (b, t), t < T, of stats (batch rows ld floats apart):
 * the four mean gradients written to gstats + b * ldg + 6 t (columns 0..3). */
int dabsn_hip_glue_rows_bwd(int64_t B, int64_t T, int64_t ld, const float* stats, int mode,
                            const float* gcocktail, float* gstats, int64_t ldg,
                            hipStream_t stream);
/* Admitted-slot selection (src/dabsn/read.py:185-239): per row, floor = cummax(adm) -
 * window (whole = 0, seq geometry) or max over the row of adm - window (whole = 1, field
 * and hybrid geometry, read.py:189-191), member = adm >= floor, order = stable partition
 * (members by ascending t, then the rest), counts = #members, rank[t] = position of t in
 * order. adm [B,T] as fp32 values; window points at an fp32 scalar (already softplus-ed).
 * adm_dtype = the dtype the admission was computed in: 1 (bf16) rounds the floor to bf16
 * as the reference's bf16 subtraction does, 0 (fp32) keeps it fp32. Bit-exact. */
int dabsn_hip_bank_select(int adm_dtype, int whole, int64_t B, int64_t T, const float* adm,
                          const float* window, int64_t* order, int64_t* counts, int32_t* rank,
                          hipStream_t stream);
/* Incremental admission for a carried bank (streaming decode; src/dabsn/memory.py:215-290
 * reruns read.py:58-72, 155-191 over the whole bank each step). In seq geometry the floor
 * of a position depends only on the positions before it, so its glue and membership are
 * final when it is appended. Per batch row, for the n positions base .. base + n - 1 of a
 * bank of capacity cap: computes their key bias, admission and cocktail from the
 * statistics rows stats [B, cap, 6] exactly as dabsn_hip_means_glue (`mode`, `params`)
 * into key_bias [B, cap], admission [B, cap] and cocktail [B, cap, 4] (16-byte aligned);
 * then, in position order, updates the running prefix max amax [B] and the member count
 * mcount [B] (fp32 / int64; both restart when base = 0), appending each member position to the row's
 * slot list members [B, cap] (int64, ascending). members[b, :mcount[b]] then equals
 * dabsn_hip_bank_select's order[b, :counts[b]] over the first base + n positions, bit for
 * bit. adm_dtype as for bank_select; window as there. With stats = NULL the admission
 * values are taken from `admission` as they stand (params, key_bias and cocktail unused).
 * base + n <= cap. */
int dabsn_hip_admit_step(int mode, int64_t B, int64_t n, int64_t base, int64_t cap,
                         const float* stats, int64_t hidden, const float* const* params,
                         const float* window, int adm_dtype, float* key_bias, float* admission,
                         float* cocktail, float* amax, int64_t* mcount, int64_t* members,
                         hipStream_t stream);

/* Successor-fold codes of a selected bank (no reference counterpart: they let the read skip
 * its successor-row products, see dabsn_hip_read3_fwd_keep). order [B,T] and counts [B]
 * as dabsn_hip_bank_select returns them; the bank's next positions are min(idx + 1, T - 1).
 * codes [B,N] (optional): 1 when slot j's next position is slot j + 1's position, 0 when it
 * is its own position or j >= counts[b], 2 otherwise. unfoldable (optional, one uint32) is
 * set to 1 when any admitted slot of any row codes 2, else 0. */
int dabsn_hip_bank_fold(int64_t B, int64_t T, int64_t N, const int64_t* order,
                        const int64_t* counts, int8_t* codes, uint32_t* unfoldable,
                        hipStream_t stream);

/* out = a + x (x may be NULL: out = a) over a [B, R, C] box of `dtype` elements whose
 * operands each have a batch and a row stride in elements (columns contiguous): a time
 * window [t0, t0 + R) of [B, T, C] tensors has strides (T C, C), a column block of a wider
 * row the row's width. bf16 sums are formed in fp32 and rounded once (torch's add). out may
 * alias a or x elementwise. No reference counterpart: it moves the windows a time-chunked
 * read hands between its pieces without a copy per operand. */
int dabsn_hip_window_add(int dtype, int64_t B, int64_t R, int64_t C, const void* a, int64_t a_sb,
                         int64_t a_sr, const void* x, int64_t x_sb, int64_t x_sr, void* out,
                         int64_t o_sb, int64_t o_sr, hipStream_t stream);
/* The width a read of a bank_select result needs (read.py:233: the host reads the largest
 * admitted count) and, with check_fold, whether the successor fold applies: out[0] (int64) =
 * max over rows of counts, out[1] = 1 when some admitted slot codes 2 in
 * dabsn_hip_bank_fold's terms, else 0. order [B,T], counts [B] as bank_select returns them;
 * order may be NULL without check_fold. One device read of out replaces the reduction, the
 * flag and their stacking. */
int dabsn_hip_bank_width(int64_t B, int64_t T, const int64_t* order, const int64_t* counts,
                         int check_fold, int64_t* out, hipStream_t stream);
/* The slot arrays of a read of width N <= T (read.py:233-239, 298-303) in one launch, all
 * [B,N]: idx = order[:, :N] (int64), valid = j < max(counts, 1) (one byte, 0/1),
 * next_idx = min(idx + 1, T - 1), read_idx = idx - query_start (int64) and, when codes is
 * not NULL, the fold codes of dabsn_hip_bank_fold (int8). */
int dabsn_hip_bank_slots(int64_t B, int64_t T, int64_t N, const int64_t* order,
                         const int64_t* counts, int64_t query_start, int64_t* idx,
                         uint8_t* valid, int64_t* next_idx, int64_t* read_idx, int8_t* codes,
                         hipStream_t stream);

/* Bank gather (read.py:241-256, 298-303): for j < N, K = w[idx]/max(|w[idx]|,eps),
 * V = w[idx], Vn = w[next_idx] ([B,N,H]). norm_w [B,T] fp32. Vn may be null (then
 * next_idx is not read): a folded read needs no successor rows. */
int dabsn_hip_bank_gather(int dtype, int64_t B, int64_t T, int64_t N, int64_t H, const void* w,
                          const float* norm_w, const int64_t* idx, const int64_t* next_idx,
                          void* K, void* V, void* Vn, hipStream_t stream);
/* Backward, as a deterministic gather over positions using rank [B,T]:
 * gw[t] = (rank[t] < N ? gV + dnorm(gK) : 0) + sum of gVn over slots whose next index is t
 * (written for every position; gVn may be null). */
int dabsn_hip_bank_gather_bwd(int dtype, int64_t B, int64_t T, int64_t N, int64_t H,
                              const void* w, const float* norm_w, const int32_t* rank,
                              const void* K, const void* gK, const void* gV, const void* gVn,
                              void* gw, hipStream_t stream);
/* The same over the first T positions of each row of a longer write tape (a bank that is the
 * prefix of the sequence, as a time-chunked read builds it): norm_w and gw rows are ldg
 * positions apart, rank is [B,T]; positions >= T are not touched. accumulate = 1 adds into
 * gw instead of writing it. */
int dabsn_hip_bank_gather_bwd_prefix(int dtype, int64_t B, int64_t T, int64_t ldg, int64_t N,
                                     int64_t H, const float* norm_w, const int32_t* rank,
                                     const void* K, const void* gK, const void* gV,
                                     const void* gVn, int accumulate, void* gw,
                                     hipStream_t stream);

/* ---- block glue (inference) ---------------------------------------------------------
 * The element work around one block's read and its MLP branch, each as one kernel, for the
 * streaming step (no backward). All tensors dense in `dtype`; every intermediate the
 * reference stores in that dtype is rounded to it here too. */
/* out = y + read_gain * (proj + long_gain * long): the read's output (read.py:435, 821:
 * out(...) + long_gain * long) fed into the block's mix (model.py:336:
 * y + read_gain * read). n elements; gains are fp32 scalars holding values of `dtype`. */
int dabsn_hip_read_mix(int dtype, int64_t n, const void* proj, const void* lng,
                       const float* long_gain, const void* y, const float* read_gain, void* out,
                       hipStream_t stream);
/* MLPRMSNorm (model.py:35-45) over rows of H: rsqrt(mean(x^2) + eps) in fp32, the
 * normalised row rounded to `dtype`, times weight [H] (same dtype). */
int dabsn_hip_rms_norm(int dtype, int64_t rows, int64_t H, const void* x, const void* weight,
                       float eps, void* out, hipStream_t stream);
/* relu(x).square() of the MLP branch (model.py:188-195); NaN stays NaN. */
int dabsn_hip_relu_square(int dtype, int64_t n, const void* x, void* out, hipStream_t stream);

/* ---- three-way admitted read ------------------------------------------------------
 * Replaces the device kernels of dabsn::admitted_three_way_read_compact_flash and
 * dabsn::_admitted_three_way_read_compact_flash_backward
 * (src/dabsn/kernels/compact_flash.py:71-107, 181-224; math admitted.py:9-239; CPU
 * cpu_runtime.cpp:321-438, 479-662). q [B,T,H] (normalised queries), K (normalised
 * keys), V, Vn [B,N,H] in `dtype`; cocktail [B,T,4], bank_cocktail [B,N,4], key_bias and
 * admission [B,N] in fp32; scale and gains[4] (short, pad, induct, cocktail) point at
 * fp32 scalars; idx [B,N] int64 and valid [B,N] uint8; mode 0 = seq (allow idx <= t,
 * induction idx < t), 1 = field (allow valid, induction idx < T-1).
 *
 * Workspace sizes by `part`: 0 = one buffer for dabsn_hip_read3_fwd, 1 = one buffer for
 * dabsn_hip_read3_bwd (which recomputes the forward), 2 = the kept part (scores, tile
 * ranges, row statistics, the read weights P_V) that dabsn_hip_read3_fwd_keep fills for
 * dabsn_hip_read3_bwd_after_fwd, 3 = the forward scratch beside it, 4 = the backward
 * scratch beside it. */
size_t dabsn_hip_read3_workspace_bytes(int dtype, int64_t B, int64_t T, int64_t N, int64_t H,
                                       int part);
int dabsn_hip_read3_fwd(int dtype, int64_t B, int64_t T, int64_t N, int64_t H, const void* q,
                        const void* K, const void* V, const void* Vn, const float* cocktail,
                        const float* bank_cocktail, const float* key_bias, const float* admission,
                        const float* scale, const int64_t* idx, const uint8_t* valid, int mode,
                        const float* const* gains, void* out, void* workspace,
                        size_t workspace_bytes, hipStream_t stream);
/* Backward: gout [B,T,H] -> gq, gK, gV, gVn (dtype), gcocktail [B,T,4], gbank_cocktail
 * [B,N,4], gkey_bias, gadmission [B,N] (fp32) and gscalars5 = (scale, short_gain,
 * pad_gain, induct_gain, cocktail_gain). */
int dabsn_hip_read3_bwd(int dtype, int64_t B, int64_t T, int64_t N, int64_t H, const void* gout,
                        const void* q, const void* K, const void* V, const void* Vn,
                        const float* cocktail, const float* bank_cocktail, const float* key_bias,
                        const float* admission, const float* scale, const int64_t* idx,
                        const uint8_t* valid, int mode, const float* const* gains, void* gq,
                        void* gK, void* gV, void* gVn, float* gcocktail, float* gbank_cocktail,
                        float* gkey_bias, float* gadmission, float* gscalars5, void* workspace,
                        size_t workspace_bytes, hipStream_t stream);
/* The forward for a caller that will run the backward on the same inputs: as
 * dabsn_hip_read3_fwd, with the workspace in two buffers. `kept` (part 2 bytes) receives
 * the scores, tile ranges, row statistics and the read weights P_V [B,T,N] (the folded
 * weights with `fold`); `scratch` (part 3 bytes) is free once the call's work has
 * completed.
 * `fold` (optional, int8 [B,N]; the successor fold): fold[b][j] in {0, 1} states that the
 * successor row of every valid slot is a bank row, Vn[j] = V[j + fold[j]] (1: slot j + 1
 * holds the next position; 0: the clamped last position, Vn[j] = V[j]). The induction
 * weights then join P_V at those columns and Vn is not read (it may be null): one product
 * in the output GEMM instead of two. The same `fold` must reach the backward. */
int dabsn_hip_read3_fwd_keep(int dtype, int64_t B, int64_t T, int64_t N, int64_t H,
                             const void* q, const void* K, const void* V, const void* Vn,
                             const float* cocktail, const float* bank_cocktail,
                             const float* key_bias, const float* admission, const float* scale,
                             const int64_t* idx, const uint8_t* valid, const int8_t* fold,
                             int mode, const float* const* gains, void* out, void* kept,
                             size_t kept_bytes, void* scratch, size_t scratch_bytes,
                             hipStream_t stream);
/* The backward without recomputing the forward's scores and row statistics: `kept` is the
 * buffer a dabsn_hip_read3_fwd_keep call on the same inputs filled; it is only read, so
 * the backward can run again on it. `scratch` holds part 4 bytes. Saves the score GEMM
 * and softmax-row pass of the recompute, and the rebuild and transpose-fold of P_V, at
 * the cost of keeping B*T*N*(4 + element size) bytes of scores and weights (plus the row
 * statistics) between forward and backward. With the forward's `fold`, Vn
 * and gVn may be null: gVn is not formed, the gradient of slot j's successor row is added
 * to gV[j + fold[j]] (no gO Vn^T and no P_Vn^T gO GEMM). */
int dabsn_hip_read3_bwd_after_fwd(int dtype, int64_t B, int64_t T, int64_t N, int64_t H,
                                  const void* gout, const void* q, const void* K, const void* V,
                                  const void* Vn, const float* cocktail,
                                  const float* bank_cocktail, const float* key_bias,
                                  const float* admission, const float* scale,
                                  const int64_t* idx, const uint8_t* valid,
                                  const int8_t* fold, int mode, const float* const* gains,
                                  void* gq, void* gK, void* gV, void* gVn, float* gcocktail,
                                  float* gbank_cocktail, float* gkey_bias, float* gadmission,
                                  float* gscalars5, const void* kept, size_t kept_bytes,
                                  void* scratch, size_t scratch_bytes, hipStream_t stream);

/* Decode read: the forward of dabsn_hip_read3_fwd (mode 0, seq) for a few query rows
 * (T <= 8) against a long bank, reading the bank in place instead of from gathered K, V,
 * Vn copies. Replaces bank gather + three-way read on the streaming path of the carried
 * memory (src/dabsn/memory.py:215-290 -> read.py:650-838), where the bank is a growing
 * buffer: bank [B, bank_ld, H] in `dtype` with the first bank_len positions per batch row
 * live (bank_ld >= bank_len), norm_w [B, bank_len] fp32 write norms, idx / next_idx
 * [B, N] int64 bank positions of the admitted slots and their successors (addressing),
 * read_idx [B, N] int64 the slots' query-relative indices (masks: allow read_idx <= t,
 * induction read_idx < t), valid [B, N] uint8; the other arguments as in
 * dabsn_hip_read3_fwd. K = normalize(write) is rounded to `dtype` as the gather stores
 * it. H % 8 == 0; q, bank and out 16-byte aligned; T * H * sizeof(dtype) <= 64 KiB;
 * B * bank_ld < 2^32. One query row (T == 1) with H <= 2048 reads the bank once (online
 * softmaxes per pathway, the P V products from the exact fp32 weights); otherwise scores,
 * softmax rows and products run as separate passes with P_V / P_Vn rounded to `dtype`.
 * Inference only: there is no backward. */
size_t dabsn_hip_read3_decode_workspace_bytes(int dtype, int64_t B, int64_t T, int64_t N,
                                              int64_t H);
int dabsn_hip_read3_decode(int dtype, int64_t B, int64_t T, int64_t N, int64_t H, const void* q,
                           const void* bank, int64_t bank_len, int64_t bank_ld,
                           const float* norm_w, const int64_t* idx, const int64_t* next_idx,
                           const int64_t* read_idx, const uint8_t* valid, const float* cocktail,
                           const float* bank_cocktail, const float* key_bias,
                           const float* admission, const float* scale,
                           const float* const* gains, void* out, void* workspace,
                           size_t workspace_bytes, hipStream_t stream);

/* The one-query decode read (T == 1, H % 8 == 0, H <= 2048) taking its slots straight from
 * a carried bank's admitted-slot lists and kept per-position glue, as the streaming step of
 * the carried memory holds them (src/dabsn/memory.py:215-290 -> read.py:185-256 and
 * :650-838: the reference gathers the admitted slots' cocktail, key bias and admission with
 * torch ops per step, then reads). Every per-position array has bank_ld positions per batch
 * row: bank [B, bank_ld, H], stats [B, bank_ld, 6] fp32 (write norm in column 5),
 * members [B, bank_ld] int64 (row b's admitted positions, ascending), cocktail
 * [B, bank_ld, 4], key_bias and admission [B, bank_ld] fp32; counts [B] int64 members per
 * row. The read covers slots j < N: slot j is members[b, j], valid below max(counts[b], 1);
 * its successor is min(idx + 1, bank_len - 1), its query-relative index idx - query_start;
 * the query's cocktail is the bank's at bank_len - 1. Equals dabsn_hip_read3_decode on
 * those arrays. N <= bank_ld; workspace: dabsn_hip_read3_decode_workspace_bytes(dtype, B,
 * 1, N, H). */
int dabsn_hip_read3_decode_members(int dtype, int64_t B, int64_t N, int64_t H, const void* q,
                                   const void* bank, int64_t bank_len, int64_t bank_ld,
                                   const float* stats, const int64_t* members,
                                   const int64_t* counts, int64_t query_start,
                                   const float* cocktail, const float* key_bias,
                                   const float* admission, const float* scale,
                                   const float* const* gains, void* out, void* workspace,
                                   size_t workspace_bytes, hipStream_t stream);

/* The decode read for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops whose buffers are all planned ahead). This entry point has no
 * counterpart in the reference. Same arguments and result as dabsn_hip_read3_decode
 * without the workspace: the library keeps a scratch array of
 * DABSN_READ3_DECODE_NOALLOC_MAX_BYTES on every device it runs on, from module load until
 * the process ends, and calls nothing that allocates. A call whose decode plan needs more
 * scratch than that returns DABSN_ERR_ARG with nothing enqueued (at H = 2048 in bf16 a
 * one-row read of batch 256 fits banks of about 10,000 slots). Calls that overlap on one
 * device -- on other streams or threads -- share the array and race; the array keeps the
 * last call's contents, none of which a later call reads. */
#define DABSN_READ3_DECODE_NOALLOC_MAX_BYTES ((size_t)128 << 20)
int dabsn_hip_read3_decode_noalloc(int dtype, int64_t B, int64_t T, int64_t N, int64_t H,
                                   const void* q, const void* bank, int64_t bank_len,
                                   int64_t bank_ld, const float* norm_w, const int64_t* idx,
                                   const int64_t* next_idx, const int64_t* read_idx,
                                   const uint8_t* valid, const float* cocktail,
                                   const float* bank_cocktail, const float* key_bias,
                                   const float* admission, const float* scale,
                                   const float* const* gains, void* out, hipStream_t stream);

/* ---- dense-mask three-way admitted read --------------------------------------------
 * Replace the device kernels of dabsn::admitted_three_way_read_native and
 * dabsn::_admitted_three_way_read_backward (src/dabsn/kernels/admitted.py:383-622; the
 * math of admitted.py:16-65 and :126-236, the CPU form three_way_read_cpu /
 * three_way_read_bwd in src/dabsn/kernels/cpu_runtime.cpp). Every float operand is fp32
 * and contiguous (the reference's compute dtype): query [B,T,H], bank_keys, bank_writes,
 * next_writes [B,N,H], cocktail [B,T,4], bank_cocktail [B,N,4], bank_key_bias and
 * bank_admission [B,N]; allow and induct_allow [B,T,N] and eligible and induct_eligible
 * [B,T] are bytes (0 / 1, torch.bool). `scalars` is a device fp32 [5] array in the op's
 * schema order: scale, short_gain, pad_gain, induct_gain, cocktail_gain. The forward
 * writes out [B,T,H]; the backward takes grad_out [B,T,H] and writes every float input's
 * gradient (g_scalars [5] in the same order). B, T, N, H > 0 (callers return empty or zero
 * results for empty shapes). Workspace: dabsn_hip_read_dense_workspace_bytes(B, T, N, H,
 * backward) bytes, owned by the call. */
size_t dabsn_hip_read_dense_workspace_bytes(int64_t B, int64_t T, int64_t N, int64_t H,
                                            int backward);
int dabsn_hip_read_dense_fwd(int64_t B, int64_t T, int64_t N, int64_t H, const float* query,
                             const float* bank_keys, const float* bank_writes,
                             const float* next_writes, const float* cocktail,
                             const float* bank_cocktail, const float* bank_key_bias,
                             const float* bank_admission, const uint8_t* allow,
                             const uint8_t* induct_allow, const uint8_t* eligible,
                             const uint8_t* induct_eligible, const float* scalars, float* out,
                             void* workspace, size_t workspace_bytes, hipStream_t stream);
/* The same read returning also its three masked softmaxes (fp32 [B, T, N] each: short,
 * permanent, induction), as the reference's 4-output operator dabsn::admitted_three_way_read
 * does (src/dabsn/kernels/admitted.py:16-65; its autograd, admitted.py:126-247, works from
 * those saved weights). The weight pointers are all given or all null. */
int dabsn_hip_read_dense_fwd_weights(int64_t B, int64_t T, int64_t N, int64_t H,
                                     const float* query, const float* bank_keys,
                                     const float* bank_writes, const float* next_writes,
                                     const float* cocktail, const float* bank_cocktail,
                                     const float* bank_key_bias, const float* bank_admission,
                                     const uint8_t* allow, const uint8_t* induct_allow,
                                     const uint8_t* eligible, const uint8_t* induct_eligible,
                                     const float* scalars, float* out, float* short_weights,
                                     float* permanent_weights, float* induct_weights,
                                     void* workspace, size_t workspace_bytes, hipStream_t stream);

int dabsn_hip_read_dense_bwd(int64_t B, int64_t T, int64_t N, int64_t H, const float* grad_out,
                             const float* query, const float* bank_keys, const float* bank_writes,
                             const float* next_writes, const float* cocktail,
                             const float* bank_cocktail, const float* bank_key_bias,
                             const float* bank_admission, const uint8_t* allow,
                             const uint8_t* induct_allow, const uint8_t* eligible,
                             const uint8_t* induct_eligible, const float* scalars, float* g_query,
                             float* g_keys, float* g_writes, float* g_next, float* g_cocktail,
                             float* g_bank_cocktail, float* g_key_bias, float* g_admission,
                             float* g_scalars, void* workspace, size_t workspace_bytes,
                             hipStream_t stream);

/* ---- permanent associative delta scan --------------------------------------------
 * Replaces dabsn::permanent_delta_scan and its registered backward
 * (src/dabsn/kernels/permanent.py:39-119, 384-433; CPU cpu_runtime.cpp:1075-1188).
 * key, value [B,T,H], beta [B,T], fp32 (the op converts other dtypes). Per batch row a
 * state S [H,H] starts at zero; out_t = S k_t, then S += beta_t (v_t - out_t) k_t^T.
 * H <= 2048. Backward: dkey, dvalue [B,T,H], dbeta [B,T] fp32 from grad_out [B,T,H]; it
 * recomputes the per-row states into the workspace, keeping every 8th one and the last
 * (dabsn_hip_permanent_scan_workspace_bytes(): 4 B (ceil(T/8)+1) H^2 bytes plus r_t and
 * partial sums), and rebuilds the states in between by undoing each step's update; the
 * reference's reverse pass keeps all T states. Results are deterministic. */
int dabsn_hip_permanent_scan_fwd(int64_t B, int64_t T, int64_t H, const float* key,
                                 const float* value, const float* beta, float* out,
                                 hipStream_t stream);
size_t dabsn_hip_permanent_scan_workspace_bytes(int64_t B, int64_t T, int64_t H);
int dabsn_hip_permanent_scan_bwd(int64_t B, int64_t T, int64_t H, const float* key,
                                 const float* value, const float* beta, const float* grad_out,
                                 float* dkey, float* dvalue, float* dbeta, void* workspace,
                                 size_t workspace_bytes, hipStream_t stream);

/* ---- local field patch gather ----------------------------------------------------
 * Replaces dabsn::local_field_gather and its registered backward
 * (src/dabsn/kernels/local_field.py:208-244; CPU cpu_runtime.cpp:1191-1237).
 * out [B,P,K,D] = x [B,N,D] gathered at patch [P,K] (int64, values in [0, N)). Backward:
 * grad_x [B,N,D] = scatter-add of grad_out [B,P,K,D], each source summed over its entries
 * p*K + j in increasing order (the reference CPU loop's order: fp32 results equal it
 * bit for bit). dtype 0 (fp32) or 1 (bf16; sums in fp32, one rounding). An index
 * outside [0, N) sets the first workspace word to 1 (its entries give zero) and the call
 * still returns DABSN_OK; the caller reads the word. Workspace:
 * dabsn_hip_local_field_workspace_bytes(N, P, K, backward). */
size_t dabsn_hip_local_field_workspace_bytes(int64_t N, int64_t P, int64_t K, int backward);
int dabsn_hip_local_field_gather(int dtype, int64_t B, int64_t N, int64_t D, int64_t P,
                                 int64_t K, const void* x, const int64_t* patch, void* out,
                                 void* workspace, size_t workspace_bytes, hipStream_t stream);
int dabsn_hip_local_field_gather_bwd(int dtype, int64_t B, int64_t N, int64_t D, int64_t P,
                                     int64_t K, const void* grad_out, const int64_t* patch,
                                     void* grad_x, void* workspace, size_t workspace_bytes,
                                     hipStream_t stream);

/* ---- chunked readout cross-entropy: row kernels ----------------------------------
 * Replace the per-chunk row math of ChunkedLinearCrossEntropy
 * (src/dabsn/runtime/loss.py:52-137): the readout GEMM stays a plain GEMM; these take its
 * logits [rows, V] (row stride ldl >= V, `dtype` 0 fp32 / 1 bf16, read as fp32) and int64
 * targets [rows]. Forward: lse [rows] = logsumexp of the row, nll [rows] = lse -
 * logit[target] (0 where target == ignore_index). Backward: dlogits [rows, V] fp32 =
 * (exp(logit - lse) - onehot(target)) * scale[0] (0 rows where ignored); scale is a device
 * fp32 scalar (grad / valid count). A target outside [0, V) other than ignore_index sets
 * *err to 1 and the row counts as ignored; the caller reads the word. */
int dabsn_hip_ce_fwd(int dtype, int64_t rows, int64_t V, const void* logits, int64_t ldl,
                     const int64_t* targets, int64_t ignore_index, float* lse, float* nll,
                     uint32_t* err, hipStream_t stream);
int dabsn_hip_ce_bwd(int dtype, int64_t rows, int64_t V, const void* logits, int64_t ldl,
                     const int64_t* targets, int64_t ignore_index, const float* lse,
                     const float* scale, float* dlogits, uint32_t* err, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DABSN_HIP_H_ */
