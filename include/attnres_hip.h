/*
 * attnres_hip.h - C ABI of the MI355X (gfx950) Fast-AttnRes read.
 *
 * One AttnRes "read" mixes S depth sources of N token rows of width D with a
 * static query q[R] (1 <= R <= D).  The key of source s at token n is the
 * last R coordinates of its value row:
 *
 *   t_s = v_s[D-R:D];  r_s = sqrt(mean(t_s^2) + eps);  z_s = scale*<t_s/r_s, q>
 *   p_s = softmax_s(z);  out = sum_s p_s * v_s
 *
 * Storage is BF16 (values, query, output, gradients); all arithmetic is FP32.
 *
 * Conventions shared by every entry point:
 *   - every pointer is a device pointer unless stated otherwise; sizes and
 *     strides are counted in ELEMENTS, not bytes;
 *   - a value row is unit-stride along D; rows of one source are
 *     `row_stride` elements apart (any int64, including > 2^31);
 *   - `stream` is a hipStream_t (passed as void* so that this header needs no
 *     HIP include); work is only enqueued on it: nothing here allocates,
 *     synchronises or reads device memory from the host, so every call may be
 *     captured into a HIP graph;
 *   - calls share no mutable state, except attnres_hip_packed_backward_noalloc,
 *     whose calls on one GPU share its device scratch array: two of them that
 *     overlap in time there (concurrent streams or threads, or two captured
 *     graphs replayed at once) race;
 *   - the return value is ATTNRES_OK or one of the codes below; arguments are
 *     fully checked on the host before anything is enqueued, so an invalid
 *     call never launches a kernel.  attnres_hip_last_error() describes the
 *     most recent failure of the calling thread.
 *
 * Saved tensors written by the forward and read by the backward:
 *   out_refine[N, D] int8, low-order correction of the BF16 output: the FP32
 *                 mix is o = bf16(o) + q * ulp(bf16(o)) / 256 to within
 *                 ulp/512 (q = 0 for |o| < 2^-111, inf and NaN).  The
 *                 backward needs <dO, o>; BF16 alone leaves an error that
 *                 accumulates in dq over tokens.
 *   logit[N, S]   FP32, already-scaled routing logit z_s per token
 *   inv_rms[N, S] FP32, 1/r_s per token
 *   stats[2, N]   FP32, row 0 = max_s z_s, row 1 = 1/sum_s exp(z_s - max)
 * The two softmax statistics are kept separate on purpose: a single FP32
 * log-sum-exp loses the normaliser when logits share an offset near 2^24.
 *
 * Save/recompute policy.  A read of at most ATTNRES_RECOMPUTE_MAX_SOURCES
 * sources need not save the output's refinement: pass out_refine = NULL to
 * the forward (nothing is stored) and out = out_refine = NULL to the plain
 * backward, which then derives delta = <dO, o> = sum_s p_s <v_s, dO> from
 * the value rows it reads anyway.  So need reads of at most
 * ATTNRES_KEYRES_MAX_SOURCES whose rows are 2048 or 4096 elements wide and
 * whose key is their last 512 or 1024, and reads of at most
 * ATTNRES_KEYRES_FULL_MAX_SOURCES of 2048-wide rows with R = D (the
 * key-resident backward keeps the key coordinates of a token's rows in
 * registers while the rows stream by).
 * attnres_hip_saves_refinement_for tells them apart; other reads must save
 * it.  (The reference makes the same structural choice with a threshold of
 * 3: recompute for S <= 3, save the FP32 mixed output for S >= 4,
 * src/attnres/_kernels/fla_full_sources.py:146-161.  Here the recompute
 * backward holds a token's rows in registers, which pays up to 6 sources.)
 */
#ifndef ATTNRES_HIP_H
#define ATTNRES_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum attnres_status {
  ATTNRES_OK = 0,
  ATTNRES_ERR_NULL_POINTER = 1,  /* a required pointer is NULL            */
  ATTNRES_ERR_SHAPE = 2,         /* S, N, D or R outside the envelope     */
  ATTNRES_ERR_STRIDE = 3,        /* a negative row or source stride       */
  ATTNRES_ERR_SCALAR = 4,        /* eps not finite-positive / scale not finite */
  ATTNRES_ERR_WORKSPACE = 5,     /* dq workspace smaller than required    */
  ATTNRES_ERR_LAUNCH = 6,        /* the HIP runtime rejected a launch     */
};

/* Envelope (the reference's package limits, src/attnres/_sources.py:12-13). */
#define ATTNRES_MAX_SOURCES 129
#define ATTNRES_MAX_WIDTH 8192
/* Reads of at most this many sources may skip the refinement (see above). */
#define ATTNRES_RECOMPUTE_MAX_SOURCES 6
/* The key-resident backward takes reads of up to this many sources with a
 * key of 512 or 1024 of 2048- or 4096-wide rows, and of up to
 * ATTNRES_KEYRES_FULL_MAX_SOURCES with the whole 2048-wide row as key (see
 * attnres_hip_saves_refinement_for). */
#define ATTNRES_KEYRES_MAX_SOURCES 16
#define ATTNRES_KEYRES_FULL_MAX_SOURCES 12

/* Element types of attnres_hip_partial_sum and attnres_hip_bank_gather. */
#define ATTNRES_DTYPE_F32 0
#define ATTNRES_DTYPE_BF16 1
/* Reads one attnres_hip_bank_gather launch takes (more take further launches). */
#define ATTNRES_MAX_GATHER_READS 48

/* Library version string; the Python package's __version__ (e.g. "2.0.1+mi355x.1"). */
const char* attnres_hip_version(void);

/* Message for the calling thread's most recent non-OK status. */
const char* attnres_hip_last_error(void);

/*
 * The library's save/recompute policy for a read of n_sources sources:
 * 1 = save (the forward stores out_refine, the backward reads out and
 * out_refine), 0 = recompute (n_sources <= ATTNRES_RECOMPUTE_MAX_SOURCES).
 * Host-only.  Replaces `_should_save_mixed` (fla_full_sources.py:146-161).
 * Reads of more sources may recompute too, depending on their shape: see
 * attnres_hip_saves_refinement_for.
 */
int attnres_hip_saves_refinement(int64_t n_sources);

/*
 * The save/recompute policy for a read of the given shape: 0 (recompute) for
 * n_sources <= ATTNRES_RECOMPUTE_MAX_SOURCES, and also for
 * n_sources <= ATTNRES_KEYRES_MAX_SOURCES when the rows are 2048 or 4096
 * elements wide and the key is their last 512 or 1024, and for
 * n_sources <= ATTNRES_KEYRES_FULL_MAX_SOURCES when width = rank = 2048 (the
 * key-resident backward: it holds the key coordinates of a token's rows and
 * takes delta from the value rows); 1 (save) otherwise.  The forward of a recomputing
 * read may pass out_refine = NULL, and its backward must then get
 * out = out_refine = NULL.  Host-only.  Replaces `_should_save_mixed`
 * (fla_full_sources.py:146-161), which keys on the source count alone.
 */
int attnres_hip_saves_refinement_for(int64_t n_sources, int64_t width, int64_t rank);

/*
 * Packed forward.  values[s, n, :] lives at values + s*source_stride +
 * n*row_stride.  Writes out[N, D] (contiguous BF16), out_refine[N, D]
 * (contiguous int8; NULL: not stored) and the saved statistics.
 *
 * Replaces the launch inside the reference op
 * `attnres::_fixed_tail_forward_with_aux` (src/attnres/_kernels/fixed_tail.py:904-960),
 * i.e. `_packed_online_forward_kernel` (fixed_tail.py:244-483).
 */
int attnres_hip_packed_forward(const void* values, int64_t source_stride,
                               int64_t row_stride, int64_t n_sources,
                               int64_t n_tokens, int64_t width,
                               const void* query, int64_t rank, float eps,
                               float scale, void* out, int8_t* out_refine,
                               float* logit, float* inv_rms, float* stats,
                               void* stream);

/*
 * Number of FP32 elements the backward needs in `dq_workspace`
 * (partial dq rows of the deterministic reduction, one per backward workgroup, plus the FP32
 * total).  Depends only on (n_tokens, width, rank); never negative for
 * in-envelope shapes, -1 otherwise.  Host-only.
 */
int64_t attnres_hip_dq_workspace_elems(int64_t n_tokens, int64_t width,
                                       int64_t rank);

/*
 * Packed backward.  Reads values (same layout as the forward), the forward's
 * out[N, D] and out_refine[N, D] (contiguous), grad_out[N, D] (contiguous
 * BF16) and the saved statistics; writes grad_values[S, N, D] (contiguous BF16) and
 * grad_query[R] (BF16).  dq is reduced over all tokens in a fixed order, so it
 * is bit-identical from run to run.  out_refine = NULL (and out ignored, may
 * be NULL) selects the recompute or key-resident kernel: the read must then
 * be one that attnres_hip_saves_refinement_for says need not save (else
 * ATTNRES_ERR_SHAPE).
 *
 * Replaces `attnres::_fixed_tail_backward` (fixed_tail.py:962-1034):
 * `_packed_online_backward_kernel` (fixed_tail.py:485-873) plus
 * `_packed_query_reduce_kernel` (fixed_tail.py:875-899) and the BF16 cast
 * (fixed_tail.py:1034).
 */
int attnres_hip_packed_backward(const void* values, int64_t source_stride,
                                int64_t row_stride, int64_t n_sources,
                                int64_t n_tokens, int64_t width,
                                const void* query, int64_t rank, float scale,
                                const void* out, const int8_t* out_refine,
                                const void* grad_out, const float* logit,
                                const float* inv_rms, const float* stats,
                                void* grad_values,
                                void* grad_query, float* dq_workspace,
                                int64_t dq_workspace_elems, void* stream);

/*
 * Packed backward that allocates nothing and takes no workspace: the same
 * arguments, kernels and results as attnres_hip_packed_backward without
 * dq_workspace / dq_workspace_elems.  The dq partial rows live in a 4 MiB
 * device array that the library holds for the life of the process, one per
 * GPU (looked up on the first call on each device, which must be current).
 * When the grid would need more partial rows than that array holds
 * ((rows + 1) * rank > 2^20 FP32 elements), the backward runs on fewer
 * workgroups: dv is the same bits, dq may differ in the FP32 order of its
 * partial sums.  rank must be at most 2^19 (always so within the envelope),
 * else ATTNRES_ERR_WORKSPACE.  Calls on one GPU share that array, so calls
 * that overlap in time on one GPU (concurrent streams, threads, or two
 * graphs captured with it replayed at once) race; calls in stream order do
 * not.  The first call on each device looks the array up
 * (hipGetSymbolAddress): make it outside stream capture; later calls make
 * only the runtime calls of every entry point (hipGetDevice, the occupancy
 * queries cached per kernel, the launches) and may be captured.
 *
 * No counterpart in the reference (its backward allocates dq partials with
 * torch.empty, fixed_tail.py:980-984).  For callers that cannot allocate
 * device memory: code under stream capture, tight serving loops, harnesses
 * that forbid hipMalloc.
 */
int attnres_hip_packed_backward_noalloc(const void* values, int64_t source_stride,
                                        int64_t row_stride, int64_t n_sources,
                                        int64_t n_tokens, int64_t width,
                                        const void* query, int64_t rank, float scale,
                                        const void* out, const int8_t* out_refine,
                                        const void* grad_out, const float* logit,
                                        const float* inv_rms, const float* stats,
                                        void* grad_values, void* grad_query, void* stream);

/*
 * Source-list forward.  `sources` and `row_strides` are HOST arrays of
 * n_sources entries: source s, row n starts at sources[s] + n*row_strides[s].
 * Sources are never packed or copied.  Same outputs as the packed forward
 * (out_refine may be NULL likewise).
 *
 * Replaces `attnres::_fixed_tail_sources_forward_with_aux`
 * (src/attnres/_kernels/fixed_tail_sources.py:78-83), i.e.
 * `_launch_standard_forward` / `_fla_standard_forward_kernel`
 * (src/attnres/_kernels/fla_full_sources.py:752-804, 297-429).
 */
int attnres_hip_sources_forward(const void* const* sources,
                                const int64_t* row_strides, int64_t n_sources,
                                int64_t n_tokens, int64_t width,
                                const void* query, int64_t rank, float eps,
                                float scale, void* out, int8_t* out_refine,
                                float* logit, float* inv_rms, float* stats,
                                void* stream);

/*
 * Source-list backward.  `sources`, `row_strides` and `grad_sources` are HOST
 * arrays of n_sources entries; grad_sources[s] is a contiguous BF16 [N, D]
 * buffer (one per list position, even when two positions hold the same
 * tensor: the caller's autograd adds them).  out_refine = NULL: the
 * recompute kernel, as for the packed backward.
 *
 * Replaces `attnres::_fixed_tail_sources_backward`
 * (fixed_tail_sources.py:85-102), i.e. `_launch_standard_backward`
 * (fla_full_sources.py:807-894): `_fla_standard_backward_kernel` (432-629)
 * and the dq reductions `_fla_standard_query_reduce_kernel` /
 * `_fla_query_reduce_kernel` (632-701).
 */
int attnres_hip_sources_backward(const void* const* sources,
                                 const int64_t* row_strides, int64_t n_sources,
                                 int64_t n_tokens, int64_t width,
                                 const void* query, int64_t rank, float scale,
                                 const void* out, const int8_t* out_refine,
                                 const void* grad_out, const float* logit,
                                 const float* inv_rms, const float* stats,
                                 void* const* grad_sources,
                                 void* grad_query, float* dq_workspace,
                                 int64_t dq_workspace_elems, void* stream);

/*
 * Accumulating backward: the same arguments as the backward above, plus
 * `accumulate`, a HOST array of n_sources flag bytes.  For a source whose
 * flag is nonzero, its gradient rows must already hold a BF16 gradient, and
 * the read's dv is added to it in the kernel (stored as bf16(old + dv), dv
 * in FP32); other sources' gradient rows are overwritten as in the plain
 * backward.  dq is written (not accumulated).  out and out_refine are
 * required (these entry points always use the saved refinement).  Several reads of the same
 * sources can so sum their source gradients without separate add kernels
 * (one extra read of the gradient rows instead of reading two buffers and
 * writing a third).
 *
 * No counterpart launch in the reference: there, autograd sums the gradients
 * of sources shared by several reads with separate add kernels after each
 * read's backward.  Used by attnres.SharedSources.
 */
int attnres_hip_packed_backward_accumulate(const void* values, int64_t source_stride,
                                           int64_t row_stride, int64_t n_sources,
                                           int64_t n_tokens, int64_t width,
                                           const void* query, int64_t rank, float scale,
                                           const void* out, const int8_t* out_refine,
                                           const void* grad_out, const float* logit,
                                           const float* inv_rms, const float* stats,
                                           void* grad_values, void* grad_query,
                                           float* dq_workspace, int64_t dq_workspace_elems,
                                           const uint8_t* accumulate, void* stream);

/*
 * Accumulating packed backward into FP32 gradient sums: as
 * attnres_hip_packed_backward_accumulate, but `grad_sums` is a contiguous FP32
 * [S, N, D] buffer and dv is written (flag 0) or added (flag nonzero) in FP32,
 * with no BF16 rounding.  For a source bank whose sources receive the sum of
 * many reads' gradients (attnres.SourceBank).  No counterpart in the reference.
 */
int attnres_hip_packed_backward_accumulate_f32(const void* values, int64_t source_stride,
                                               int64_t row_stride, int64_t n_sources,
                                               int64_t n_tokens, int64_t width,
                                               const void* query, int64_t rank, float scale,
                                               const void* out, const int8_t* out_refine,
                                               const void* grad_out, const float* logit,
                                               const float* inv_rms, const float* stats,
                                               float* grad_sums, void* grad_query,
                                               float* dq_workspace, int64_t dq_workspace_elems,
                                               const uint8_t* accumulate, void* stream);

int attnres_hip_sources_backward_accumulate(const void* const* sources,
                                            const int64_t* row_strides, int64_t n_sources,
                                            int64_t n_tokens, int64_t width,
                                            const void* query, int64_t rank, float scale,
                                            const void* out, const int8_t* out_refine,
                                            const void* grad_out, const float* logit,
                                            const float* inv_rms, const float* stats,
                                            void* const* grad_sources,
                                            void* grad_query, float* dq_workspace,
                                            int64_t dq_workspace_elems,
                                            const uint8_t* accumulate, void* stream);

/*
 * Source-list form of attnres_hip_packed_backward_accumulate_f32:
 * `grad_sums` is a HOST array of n_sources pointers to contiguous FP32 [N, D]
 * buffers (for a source bank whose reads take some slots as a list: the
 * Block schedule's completed blocks plus the running partial).  No
 * counterpart in the reference; used by attnres.SourceBank.
 */
int attnres_hip_sources_backward_accumulate_f32(const void* const* sources,
                                                const int64_t* row_strides, int64_t n_sources,
                                                int64_t n_tokens, int64_t width,
                                                const void* query, int64_t rank, float scale,
                                                const void* out, const int8_t* out_refine,
                                                const void* grad_out, const float* logit,
                                                const float* inv_rms, const float* stats,
                                                float* const* grad_sums,
                                                void* grad_query, float* dq_workspace,
                                                int64_t dq_workspace_elems,
                                                const uint8_t* accumulate, void* stream);

/*
 * Coefficient backward (a source bank's first backward stage): the same
 * arguments as attnres_hip_packed_backward / attnres_hip_sources_backward
 * (out and out_refine required), but instead of gradient rows it writes
 * coef[3, S, N] (FP32, contiguous): for token n and source s the terms of
 * dv = p dO + a q + b v (b on the key coordinates), i.e.
 *   p = exp(z - max) / sum,  a = inv_rms * scale * dz,  b = -inv_rms^2 * dz * z / R,
 *   dz = p (<v, dO> - <dO, o>);
 * dq is written as usual.  The source gradients are formed later, per source,
 * by attnres_hip_bank_gather from the dO and coefficients of every read that
 * saw it.  No counterpart in the reference; used by attnres.SourceBank.
 */
int attnres_hip_packed_backward_coef(const void* values, int64_t source_stride,
                                     int64_t row_stride, int64_t n_sources,
                                     int64_t n_tokens, int64_t width,
                                     const void* query, int64_t rank, float scale,
                                     const void* out, const int8_t* out_refine,
                                     const void* grad_out, const float* logit,
                                     const float* inv_rms, const float* stats, float* coef,
                                     void* grad_query, float* dq_workspace,
                                     int64_t dq_workspace_elems, void* stream);

int attnres_hip_sources_backward_coef(const void* const* sources,
                                      const int64_t* row_strides, int64_t n_sources,
                                      int64_t n_tokens, int64_t width,
                                      const void* query, int64_t rank, float scale,
                                      const void* out, const int8_t* out_refine,
                                      const void* grad_out, const float* logit,
                                      const float* inv_rms, const float* stats, float* coef,
                                      void* grad_query, float* dq_workspace,
                                      int64_t dq_workspace_elems, void* stream);

/* One read that saw the gathered source (attnres_hip_bank_gather). */
typedef struct attnres_gather_read {
  const void* grad_out;   /* [N, D] BF16, contiguous: the read's upstream gradient     */
  const void* query_row;  /* [D] BF16: its query on the last `rank` coordinates, 0 before */
  const float* coef;      /* [3, n_sources, N] from the read's coefficient backward   */
  int64_t n_sources;      /* the read's source count                                  */
  int64_t position;       /* the gathered source's position in the read's list        */
  int64_t rank;           /* the read's query length R                                */
} attnres_gather_read;

/*
 * Gradient of one source from every read that saw it (HOST array `reads`):
 *   grad[n] (+)= sum_r p_r dO_r[n] + a_r q_r + b_r v[n]   (b_r on r's key coordinates)
 * with p, a, b of read r at token n from its coefficient backward -- the
 * read's own dv, summed over the reads in FP32.
 * `values` are the source's BF16 rows (row n at values + n*row_stride), grad
 * is contiguous [N, D] of `grad_dtype`: ATTNRES_DTYPE_F32 (accumulate != 0
 * adds to it), or ATTNRES_DTYPE_BF16 -- the FP32 sum rounded once to BF16
 * (nearest even), for a BF16 source; this needs one launch: accumulate == 0,
 * at most ATTNRES_MAX_GATHER_READS reads, all of one rank (else
 * ATTNRES_ERR_SHAPE).  One pass over the dO rows instead of one
 * read-modify-write of an FP32 sum per read.  No counterpart in the
 * reference; used by attnres.SourceBank.
 */
int attnres_hip_bank_gather(const void* values, int64_t row_stride, int64_t n_tokens,
                            int64_t width, const attnres_gather_read* reads,
                            int64_t n_reads, void* grad, int grad_dtype, int accumulate,
                            void* stream);

/*
 * Block-schedule partial sum: out[i] = prev[i] + emitted[i] (FP32 arithmetic,
 * stored as `dtype`, ATTNRES_DTYPE_F32 or ATTNRES_DTYPE_BF16) and
 * out_bf16[i] = bf16(out[i]) (round to nearest even), for n_elems contiguous
 * elements.  The running partial of a block and its BF16 copy for the next
 * read in one pass, instead of an add, then a conversion inside the read's
 * caller.  Replaces the caller step `partial_value = partial_value + emitted`
 * followed by the read's BF16 cast (reference benchmarks/model.py:333 and
 * :279-291).
 */
int attnres_hip_partial_sum(const void* prev, const void* emitted, int dtype,
                            int64_t n_elems, void* out, void* out_bf16, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ATTNRES_HIP_H */
