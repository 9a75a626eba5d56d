/*
 * sft_ft.h -- C ABI of the MI355X (gfx950) sparse feature-transformer library
 * (libsft_ft.so).
 *
 * The library replaces the two TileLang kernels and their loader behind the
 * reference's SparseLinearFunction (rgodha24/stockfish-trainer,
 * src/model/modules/feature_transformer/, abbreviated FT/ below) and adds the
 * int16 quantized inference forward.
 *
 * Conventions shared by every entry point:
 *   - All tensor pointers are device pointers (hipMalloc / torch CUDA tensors),
 *     dense row-major.  Scalars are passed by value.  `stream` is a hipStream_t
 *     passed as void* (NULL = the null stream); all work is enqueued on it, in
 *     stream order, with no host synchronisation and no device allocation.
 *   - idx is int32 [batch, max_active]; -1 marks an inactive slot anywhere in a
 *     row (FT/kernel.py:97-98).  Values outside [0, num_inputs) other than -1
 *     (undefined behaviour in the reference) are treated as inactive, so a bad
 *     index can never address memory outside the tables.
 *   - Return value: SFT_OK (0) or a negative SFT_E* code.  Arguments are
 *     validated on the host before anything is launched; on error nothing is
 *     enqueued and sft_last_error() returns a message (thread-local).
 *   - Entry points are reentrant and may be called from any host thread.
 */
#ifndef SFT_FT_H
#define SFT_FT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SFT_ABI_VERSION 1

#define SFT_OK 0
#define SFT_EINVAL (-1)     /* null pointer, size or range out of bounds        */
#define SFT_EWORKSPACE (-2) /* workspace missing or smaller than required       */
#define SFT_EHIP (-3)       /* HIP runtime error while enqueueing               */
#define SFT_EUNSUPPORTED (-4)

/* sft_ft_fwd_f32_ex flags */
#define SFT_FWD_AUTO 0x0u /* tiled gather when the shape allows it and the workspace
                             suffices, otherwise the row gather               */
#define SFT_FWD_ROWS 0x1u /* always the row gather (workspace unused)        */

/* sft_ft_bwd_f32 flags */
#define SFT_BWD_ACCUMULATE 0x0u /* dW[f] += ..., db += ...  (reference semantics)  */
#define SFT_BWD_OVERWRITE 0x1u  /* every row of dW and all of db are written      */
#define SFT_BWD_SORTED 0x00u    /* stable sort by feature + per-feature row sum;
                                   deterministic, reference summation order     */
#define SFT_BWD_ATOMIC 0x10u    /* position-major scatter with fp32 atomics;
                                   order of the adds is not deterministic       */
#define SFT_BWD_ROWS 0x2u       /* sorted algorithm with whole-row gathers only
                                   (no column tiling); same results            */
#define SFT_BWD_PREPARED 0x20u  /* sizes: the workspace of sft_ft_bwd_f32_prepared,
                                   without the sort the prepared buffer holds  */

/* sft_ft_fwd_i16 flags */
#define SFT_Q16_ACC32 0x0u  /* exact int32 accumulation, then clamp            */
#define SFT_Q16_WRAP16 0x1u /* int16 accumulator with wrapping adds, then clamp */
#define SFT_Q16_ROWS 0x2u   /* sft_ft_fwd_i16_ex: always the row gather          */

/* Version of this ABI (SFT_ABI_VERSION of the header the library was built with). */
int sft_abi_version(void);

/* Message for the last non-zero return on the calling thread ("" if none). */
const char *sft_last_error(void);

/*
 * fp32 forward: out[b, c] = bias[c] + sum_{k active} weight[idx[b, k], c],
 * added bias first then k ascending in binary32 (the reference order).
 * Overwrites out [batch, output_size].
 * Replaces make_sparse_input_linear_forward_kernel(K, L)(idx, W, b, out)
 * (FT/kernel.py:301-312) and the TileLang kernel it runs (FT/kernel.py:66-105).
 */
int sft_ft_fwd_f32(const int32_t *idx, int64_t batch, int32_t max_active, const float *weight,
                   int64_t num_inputs, int32_t output_size, const float *bias, float *out,
                   void *stream);

/*
 * Bytes of device workspace sft_ft_fwd_f32_ex uses for these sizes and flags
 * (0 when the shape runs the row gather).  Host-only computation.
 * No reference counterpart (the reference kernel takes no workspace).
 */
int sft_ft_fwd_f32_workspace_size(int64_t batch, int32_t max_active, int64_t num_inputs,
                                  int32_t output_size, uint32_t flags, size_t *bytes);

/*
 * fp32 forward with a workspace: same result, bit for bit, as sft_ft_fwd_f32.
 * With SFT_FWD_AUTO and a workspace of sft_ft_fwd_f32_workspace_size() bytes
 * (256-byte aligned), the table is first copied into 32-column tiles in the
 * workspace (each closed by a pad row of -0.0), the index rows are compacted
 * once into per-position lists ordered by active count, and the tiles are
 * gathered one by one, each from one XCD's L2.
 * Replaces the same reference call as sft_ft_fwd_f32
 * (FT/kernel.py:301-312, 66-105).
 */
int sft_ft_fwd_f32_ex(const int32_t *idx, int64_t batch, int32_t max_active, const float *weight,
                      int64_t num_inputs, int32_t output_size, const float *bias, float *out,
                      void *workspace, size_t workspace_bytes, uint32_t flags, void *stream);

/*
 * Bytes of device workspace sft_ft_bwd_f32 needs for these sizes and flags.
 * Host-only computation.
 * No reference counterpart: the reference takes its temporaries from torch
 * inside the call (FT/kernel.py:108-138).
 */
int sft_ft_bwd_f32_workspace_size(int64_t batch, int32_t max_active, int64_t num_inputs,
                                  int32_t output_size, uint32_t flags, size_t *bytes);

/*
 * fp32 backward:
 *   weight_grad[f, :] (+)= sum over slots (b, k) with idx[b, k] == f of grad_out[b, :]
 *   bias_grad[:]      (+)= sum_b grad_out[b, :]
 * With SFT_BWD_ACCUMULATE (reference semantics, FT/kernel.py:183-186,269) rows of
 * features that do not occur are left untouched; with SFT_BWD_OVERWRITE they are
 * zeroed, so the caller needs no zero-fill.
 * workspace must hold sft_ft_bwd_f32_workspace_size(...) bytes (256-byte aligned).
 * Replaces make_sparse_input_linear_backward_kernel(K, L)(idx, dW, db, grad_out)
 * (FT/kernel.py:315-319, 255-283) with its prep (FT/kernel.py:108-138) and
 * TileLang kernel (FT/kernel.py:141-188).
 */
int sft_ft_bwd_f32(const int32_t *idx, int64_t batch, int32_t max_active, const float *grad_out,
                   int64_t num_inputs, int32_t output_size, float *weight_grad, float *bias_grad,
                   void *workspace, size_t workspace_bytes, uint32_t flags, void *stream);

/*
 * The backward's sort, run ahead under the forward.  The sort of the slots by
 * feature and its segment starts depend on the indices only, so
 * sft_ft_fwd_f32_prep sorts them into a prepared buffer on a side stream while
 * its forward kernels run (joined before it returns), and
 * sft_ft_bwd_f32_prepared takes that buffer instead of sorting: its critical
 * path is the bias pass and the gathers alone.  Results are those of
 * sft_ft_fwd_f32_ex and sft_ft_bwd_f32, bit for bit.  The buffer must be
 * filled with the same indices, sizes and backward flags that the prepared
 * backward is called with; the backward only reads it, so it may be read by
 * more than one backward (a graph's backward run again with retain_graph).
 * For rows narrow against their slot count (max_active >= output_size / 5)
 * the forward runs only the sort's first (radix) pass into the buffer and the
 * backward sorts the buckets beside its bias pass, into its workspace.
 * No reference counterpart: the reference sorts inside the backward
 * (FT/kernel.py:108-138), which this splits off its call
 * (FT/functions.py:12-48 forward, :50-72 backward).
 */
/* Bytes of the prepared buffer: 0 when the backward sorts nothing, or when
 * sorting under the forward would cost more than it saves (the sort grows with
 * max_active, the backward's bias pass it would otherwise run beside with
 * output_size: prepared from max_active >= output_size / 20).  With 0 bytes the
 * prepared calls behave as sft_ft_fwd_f32_ex and sft_ft_bwd_f32. */
int sft_ft_bwd_f32_prep_size(int64_t batch, int32_t max_active, int64_t num_inputs,
                             int32_t output_size, uint32_t bwd_flags, size_t *bytes);
/* sft_ft_fwd_f32_ex, and the backward's sort into prep (256-byte aligned). */
int sft_ft_fwd_f32_prep(const int32_t *idx, int64_t batch, int32_t max_active, const float *weight,
                        int64_t num_inputs, int32_t output_size, const float *bias, float *out,
                        void *workspace, size_t workspace_bytes, uint32_t flags, void *prep,
                        size_t prep_bytes, uint32_t bwd_flags, void *stream);
/* sft_ft_bwd_f32 from a prepared buffer; workspace of
 * sft_ft_bwd_f32_workspace_size(..., flags | SFT_BWD_PREPARED) bytes.  The
 * buffer is not written.  When the prepared sort is in position chunks (the
 * tiled gather at batch > 32768), weight_grad must be 16-byte aligned
 * (SFT_EINVAL otherwise: the row gather the unaligned grad would need sorts in
 * one chunk); grad_out and bias_grad may have any 4-byte alignment. */
int sft_ft_bwd_f32_prepared(const int32_t *idx, int64_t batch, int32_t max_active,
                            const float *grad_out, int64_t num_inputs, int32_t output_size,
                            float *weight_grad, float *bias_grad, void *prep, size_t prep_bytes,
                            void *workspace, size_t workspace_bytes, uint32_t flags, void *stream);

/*
 * int16 quantized inference forward (no reference counterpart: the reference's
 * int16 inference lives in its empty `stockfish` submodule; the weights come
 * from the export scaling of src/model/quantize.py:76-93):
 *   acc[b, c]      = bias[c] + sum_{k active} weight[idx[b, k], c]     (int32, exact)
 *   out[b, c]      = clamp(flags & SFT_Q16_WRAP16 ? (int16)acc : acc, clip_lo, clip_hi)
 *   psqt_out[b, p] = sum_{k active} psqt_weight[idx[b, k], p]         (int32)
 * psqt_weight/psqt_out may both be NULL (psqt_size ignored).
 * Requires max_active < 65536 so the int32 sum cannot overflow.
 */
int sft_ft_fwd_i16(const int32_t *idx, int64_t batch, int32_t max_active, const int16_t *weight,
                   int64_t num_inputs, int32_t output_size, const int16_t *bias,
                   const int32_t *psqt_weight, int32_t psqt_size, int16_t *out,
                   int32_t *psqt_out, int32_t clip_lo, int32_t clip_hi, uint32_t flags,
                   void *stream);

/*
 * Bytes of device workspace sft_ft_fwd_i16_ex uses (0 when the shape runs the
 * row gather): the packed tiles, which grow with psqt_size (the PSQT columns
 * are stored beside the int16 columns, so query with the psqt_size of the
 * call), then the rank lists of the batch.  Host-only computation.  No
 * reference counterpart.
 */
int sft_ft_fwd_i16_workspace_size(int64_t batch, int32_t max_active, int64_t num_inputs,
                                  int32_t output_size, int32_t psqt_size, uint32_t flags,
                                  size_t *bytes);

/*
 * int16 forward with a workspace: same results, bit for bit, as sft_ft_fwd_i16.
 * Unless SFT_Q16_ROWS is set, shapes with output_size % 8 == 0, at least 8
 * column tiles of 64 and psqt_size <= 8 copy the table, with the PSQT columns
 * appended to each row, into 64-column tiles in the workspace and gather them
 * XCD by XCD from L2, reading the index rows as rank lists built once in the
 * workspace (as sft_ft_fwd_i16_packed_ex).
 */
int sft_ft_fwd_i16_ex(const int32_t *idx, int64_t batch, int32_t max_active,
                      const int16_t *weight, int64_t num_inputs, int32_t output_size,
                      const int16_t *bias, const int32_t *psqt_weight, int32_t psqt_size,
                      int16_t *out, int32_t *psqt_out, int32_t clip_lo, int32_t clip_hi,
                      void *workspace, size_t workspace_bytes, uint32_t flags, void *stream);

/*
 * The int16 forward that allocates nothing, sft_ft_fwd_i16_noalloc, is in its
 * own library, libsft_ft_noalloc.so (sft_ft_noalloc.h): its static device
 * scratch is reserved only in processes that load that library.
 */

/*
 * ---- int16 table packed once, forward of one or both perspectives ----
 * No reference counterpart (the engine's int16 accumulator; the reference
 * ships none).  For inference over a fixed exported table: the 64-column tiles
 * with the PSQT columns appended, which sft_ft_fwd_i16_ex rebuilds in its
 * workspace on every call, are built once by sft_ft_i16_pack and reused.
 *
 * Bytes of the packed table.  SFT_EUNSUPPORTED unless output_size % 8 == 0,
 * output_size > 448 (at least 8 tiles of 64 columns), psqt_size <= 8 and
 * num_inputs * 128 <= 64 MiB.
 * Host-only computation.
 */
int sft_ft_i16_packed_size(int64_t num_inputs, int32_t output_size, int32_t psqt_size, size_t *bytes);

/*
 * Packs weight int16 [num_inputs, output_size] (16-byte aligned) and
 * psqt_weight int32 [num_inputs, psqt_size] (NULL exactly when psqt_size == 0)
 * into packed (256-byte aligned, packed_bytes >= sft_ft_i16_packed_size()).
 * The packed table holds copies: repack after the weights change.
 */
int sft_ft_i16_pack(const int16_t *weight, int64_t num_inputs, int32_t output_size,
                    const int32_t *psqt_weight, int32_t psqt_size, void *packed,
                    size_t packed_bytes, void *stream);

/*
 * Forward from a packed table: for each given perspective p, out_p and
 * psqt_out_p as sft_ft_fwd_i16 computes them from idx_p (bit for bit).  idx1
 * NULL: one perspective (out1, psqt_out1 unused); otherwise both perspectives
 * in one launch, sharing each tile while it is in L2.  num_inputs, output_size
 * and psqt_size must be those the table was packed with; psqt_out_p are
 * required when psqt_size > 0.  flags: SFT_Q16_WRAP16 or 0.  bias and outputs
 * 16-byte aligned.
 */
int sft_ft_fwd_i16_packed(const int32_t *idx0, const int32_t *idx1, int64_t batch,
                          int32_t max_active, const void *packed, size_t packed_bytes,
                          int64_t num_inputs, int32_t output_size, const int16_t *bias,
                          int32_t psqt_size, int16_t *out0, int16_t *out1, int32_t *psqt_out0,
                          int32_t *psqt_out1, int32_t clip_lo, int32_t clip_hi, uint32_t flags,
                          void *stream);

/*
 * Bytes of device workspace sft_ft_fwd_i16_packed_ex uses for a batch of
 * `perspectives` (1 or 2) index matrices [batch, max_active]: the per-call
 * rank lists of the gather.  Host-only computation.
 */
int sft_ft_fwd_i16_packed_workspace_size(int64_t batch, int32_t max_active, int32_t perspectives,
                                         size_t *bytes);

/*
 * sft_ft_fwd_i16_packed with a workspace (256-byte aligned, at least
 * sft_ft_fwd_i16_packed_workspace_size() bytes): the same arguments, checks and
 * results, bit for bit.  Each perspective's index rows are turned once into
 * lists ranked by active count (16-bit entries for tables of up to 65 535
 * rows), which every column tile pass then reads, instead of compacting the
 * index rows again for each tile.  No reference counterpart.
 */
int sft_ft_fwd_i16_packed_ex(const int32_t *idx0, const int32_t *idx1, int64_t batch,
                             int32_t max_active, const void *packed, size_t packed_bytes,
                             int64_t num_inputs, int32_t output_size, const int16_t *bias,
                             int32_t psqt_size, int16_t *out0, int16_t *out1, int32_t *psqt_out0,
                             int32_t *psqt_out1, int32_t clip_lo, int32_t clip_hi, void *workspace,
                             size_t workspace_bytes, uint32_t flags, void *stream);

/*
 * ---- Composed table, both perspectives in one call ----
 * The table is num_blocks (1..4) row blocks concatenated in order (the feature
 * sets of a composed transformer, FEAT/composed.py:49-50).  Block s has
 * block_rows[s] rows; when block_virtual_rows[s] > 0 it also has a virtual
 * table and its merged row r is weight_s[r] + virtual_s[r % block_virtual_rows[s]]
 * (HalfKAv2_hm's weight + virtual_weight.repeat(32, 1), FEAT/halfka_v2_hm.py:69-70;
 * block_rows[s] must be a multiple of block_virtual_rows[s]).  num_inputs is the
 * sum of block_rows.
 *
 * Bytes of workspace the forward and the backward pair calls need.  Returns
 * SFT_EUNSUPPORTED (nothing is launched by the pair calls) unless
 * output_size % 4 == 0, output_size >= 256 and num_inputs * 128 <= 64 MiB; the
 * caller then materialises the table and uses sft_ft_fwd_f32_ex / sft_ft_bwd_f32.
 * Host-only computation.  No reference counterpart.
 */
int sft_ft_pair_workspace_size(int64_t batch, int32_t max_active, int32_t num_blocks,
                               const int64_t *block_rows, const int64_t *block_virtual_rows,
                               int32_t output_size, size_t *fwd_bytes, size_t *bwd_bytes);

/*
 * Forward of both perspectives over the composed table:
 *   out0 = fwd(idx0, merged, bias), out1 = fwd(idx1, merged, bias)
 * with merged as above, each bit for bit as sft_ft_fwd_f32 on the materialised
 * table.  The merged table is built once, directly in the 32-column tiles of
 * the workspace (the table itself is never written).  Pointers 16-byte aligned.
 * Replaces ComposedFeatureTransformer.forward (FEAT/composed.py:49-54): its
 * merged_weight (FEAT/halfka_v2_hm.py:69-70, FEAT/full_threats.py:27-28, torch.cat)
 * and its two SparseLinearFunction.apply calls (FT/functions.py:12-48).
 */
int sft_ft_fwd_pair_f32(const int32_t *idx0, const int32_t *idx1, int64_t batch, int32_t max_active,
                        int32_t num_blocks, const float *const *block_weight,
                        const float *const *block_virtual, const int64_t *block_rows,
                        const int64_t *block_virtual_rows, int32_t output_size, const float *bias,
                        float *out0, float *out1, void *workspace, size_t workspace_bytes,
                        void *stream);

/*
 * Backward of the pair (overwrites every output):
 *   block_weight_grad[s] = rows of dW_0 + dW_1 for block s, where dW_p is the
 *                          reference-order weight grad of perspective p (as
 *                          sft_ft_bwd_f32 computes it, bit for bit) and the sum is
 *                          one binary32 add, as autograd sums the two grads;
 *   block_virtual_grad[s] = sum over repeats i of block_weight_grad[s][i * V + j]
 *                          (blocks with virtual rows; NULL entries otherwise);
 *   bias_grad             = sum_b grad0[b] + sum_b grad1[b].
 * Replaces the backward of the same composition: FT/functions.py:50-72 twice,
 * autograd's sum of the two table grads, the cat split and repeat's reduction.
 */
int sft_ft_bwd_pair_f32(const int32_t *idx0, const int32_t *idx1, int64_t batch, int32_t max_active,
                        const float *grad0, const float *grad1, int32_t num_blocks,
                        const int64_t *block_rows, const int64_t *block_virtual_rows,
                        int32_t output_size, float *const *block_weight_grad,
                        float *const *block_virtual_grad, float *bias_grad, void *workspace,
                        size_t workspace_bytes, void *stream);

/*
 * ---- Composed table + post-FT epilogue, both perspectives ----
 * NNUEModel._transform_inputs (src/model/model.py:86-115) on top of the
 * composed forward above, with L1 = l1 and P = output_size - l1 PSQT columns:
 *   pw_p  = clamp(x_p[:, :L1/2], 0, 1) * clamp(x_p[:, L1/2:L1], 0, 1)  (x_p: FT output of
 *           perspective p, white = idx0, black = idx1)
 *   l0    = cat(where(us, pw_white, pw_black), where(us, pw_black, pw_white)) * 127/128
 *   psqt  = (x_white[b, L1 + k] - x_black[b, L1 + k]) * (us[b] - 0.5), k = psqt_indices[b]
 * us is float [batch] (nonzero: white to move), psqt_indices int64 [batch]
 * (an index outside [0, P) gives psqt 0 and no PSQT grad).  The FT outputs
 * themselves are never written: the forward keeps the pre-activations of both
 * perspectives in `saved` (an opaque buffer the caller holds until the
 * backward), and the backward turns grad_l0 / grad_psqt straight into the
 * weight, virtual and bias grads.  Every value is bit-identical to the
 * reference ops run on the composed forward (elementwise ops in autograd's
 * order); the virtual and bias grads are fixed-order sums (<= 1e-5 of binary64).
 * Requires l1 % 8 == 0, 0 < l1 < output_size, the shape conditions of
 * sft_ft_pair_workspace_size, and 16-byte aligned l0 / grad_l0.
 */
int sft_ft_transform_workspace_size(int64_t batch, int32_t max_active, int32_t num_blocks,
                                    const int64_t *block_rows, const int64_t *block_virtual_rows,
                                    int32_t output_size, int32_t l1, size_t *saved_bytes,
                                    size_t *fwd_bytes, size_t *bwd_bytes);

/* Replaces src/model/model.py:86-115 with the composed forward it calls
   (FEAT/composed.py:49-54, FT/functions.py:12-48). */
int sft_ft_fwd_transform_f32(const int32_t *idx0, const int32_t *idx1, int64_t batch,
                             int32_t max_active, int32_t num_blocks,
                             const float *const *block_weight, const float *const *block_virtual,
                             const int64_t *block_rows, const int64_t *block_virtual_rows,
                             int32_t output_size, int32_t l1, const float *bias, const float *us,
                             const int64_t *psqt_indices, float *l0, float *psqt, void *saved,
                             size_t saved_bytes, void *workspace, size_t workspace_bytes,
                             void *stream);

/* Backward of the same (autograd through src/model/model.py:93-115 and the
   composed backward, FT/functions.py:50-72); overwrites every grad output. */
int sft_ft_bwd_transform_f32(const int32_t *idx0, const int32_t *idx1, int64_t batch,
                             int32_t max_active, const float *grad_l0, const float *grad_psqt,
                             const float *us, const int64_t *psqt_indices, const void *saved,
                             size_t saved_bytes, int32_t num_blocks, const int64_t *block_rows,
                             const int64_t *block_virtual_rows, int32_t output_size, int32_t l1,
                             float *const *block_weight_grad, float *const *block_virtual_grad,
                             float *bias_grad, void *workspace, size_t workspace_bytes,
                             void *stream);

/*
 * Ranger22 parameter update of one table (or any fp32 tensor), in place:
 *   variance_ma = variance_ma * beta2 + (grad * grad) * (1 - beta2)
 *   grad_ma_cur = grad_ma_cur * beta1^2 + grad * (1 - beta1^2)
 *   c           = two_nl_factor * (1 - 1 / (||p_row||_2 + eps))   (p before the update)
 *   p           = p * (1 - lr * c)
 *                 - ((grad_ma_cur * pnm_a + grad_ma_prev * pnm_b) * noise_norm_recip
 *                    / (sqrt(variance_ma) * inv_sqrt_bc2 + eps)) * step_size
 * p, grad and the states are [rows, cols] row-major; the norm is per row
 * (a 1-D tensor is passed as rows = 1).  scalars is a device array of 12
 * floats in the reference's order: lr, inv_sqrt_bc2, eps, two_nl_factor,
 * noise_norm_recip, pnm_a, pnm_b, step_size, beta2, 1 - beta2, beta1^2,
 * 1 - beta1^2.  Each element's operations round to binary32 in this order (no
 * FMA contraction); the row norm is a fixed-order fp32 sum.
 * Replaces the torch.compile'd full update of Ranger22
 * (src/ranger22/optimizer.py:46-77 for 1-D, :80-111 for 2-D tensors), called
 * from Ranger22.step (src/ranger22/optimizer.py:472-480).
 */
int sft_ranger22_update_f32(float *p, const float *grad, float *variance_ma, float *grad_ma_cur,
                            const float *grad_ma_prev, int64_t rows, int64_t cols,
                            const float *scalars, void *stream);

/*
 * ---- Feature-index encoder ----
 * Positions -> the FT's index rows of both perspectives, in the reference's
 * order (FeatureSet::fill_feature_indices_sparse and
 * fill_row_from_position_without_values, src/rust/feature_extraction.rs:209-236,
 * 442-477; HalfKAv2_hm :389-402, 677-685; Full_Threats :572-675, 687-833).
 *   boards:       uint8 [batch][64], piece id per square (a1 = 0 .. h8 = 63;
 *                 id = 2 * type + color, pawn..king = 0..5, white = 0; 255 empty)
 *   side_to_move: uint8 [batch], 0 = white
 *   components:   host array of SFT_FEATURES_* in feature-set order, e.g.
 *                 {SFT_FEATURES_THREATS, SFT_FEATURES_HALFKA} = "Full_Threats+HalfKAv2_hm"
 *   white_indices / black_indices: int32 [batch][max_active], max_active = the
 *                 components' maxima summed (128 threats, 32 HalfKAv2_hm); each
 *                 component's features follow the previous one's, offset by its
 *                 input count; -1 after the last
 *   us (float), psqt_indices, layer_stack_indices (int64): [batch], optional
 *                 (NULL): 1.0 for white to move, (pieces - 1) / 4
 *   white_count / black_count: int32 [batch], optional: features found per
 *                 row; above a component's maximum the row keeps the first ones
 * Positions need one king per side and no pawn on the first or last rank (as
 * any chess position); other boards give unspecified rows, never a fault.
 */
#define SFT_FEATURES_THREATS 1
#define SFT_FEATURES_HALFKA 2
int sft_encode_features(const uint8_t *boards, const uint8_t *side_to_move, int64_t batch,
                        const int32_t *components, int32_t num_components, int32_t *white_indices,
                        int32_t *black_indices, int32_t max_active, float *us,
                        int64_t *psqt_indices, int64_t *layer_stack_indices,
                        int32_t *white_count, int32_t *black_count, void *stream);

/*
 * ---- .nnue export: signed LEB128 ----
 * Encodes n signed integers (elem_bytes 1, 2 or 4: int8 / int16 / int32) as the
 * concatenation of their signed LEB128 codes, in element order, into out
 * (device, out_capacity >= n * 2 / 3 / 5 bytes), and the byte count into
 * *out_len (a device int64, written by the last kernel on the stream).
 * Replaces _encode_leb_128_array (src/scripts/serialize.py:61-93), the
 * payload of _write_leb_128_array (:254-257) for the FT bias, weights and PSQT
 * weights of the .nnue file.
 */
int sft_leb128_workspace_size(int64_t n, size_t *bytes);
int sft_leb128_encode(const void *values, int32_t elem_bytes, int64_t n, uint8_t *out,
                      size_t out_capacity, int64_t *out_len, void *workspace,
                      size_t workspace_bytes, void *stream);

/*
 * Export quantization on the device (src/model/quantize.py:83-84):
 * out[i] = round_half_even(float32(x[i] * scale)) saturated to int16.
 * No reference counterpart as a kernel (the reference runs it as torch ops).
 */
int sft_quantize_i16(const float *x, int64_t n, float scale, int16_t *out, void *stream);

/*
 * Measurement helper (no reference counterpart): one dispatch of `blocks`
 * 256-thread workgroups whose 8-lane groups each gather 8 * rounds 128-byte rows
 * of table (table_rows x 128 bytes, table_rows a power of two <= 2^24, 16-byte
 * aligned) at pseudo-random row numbers, writing one 16-byte sum per thread to
 * out (out_bytes >= blocks * 4096).  Bytes gathered = blocks * 32 * 8 * rounds
 * * 128.  With a table that fits one XCD's L2 it measures the attainable rate of
 * the L2-served row gathers the tiled FT kernels make (timed as
 * "probe_l2_gather" by sft_prof_*).
 */
int sft_probe_l2_gather(const float *table, int64_t table_rows, int32_t rounds, int32_t blocks,
                        float *out, size_t out_bytes, void *stream);

/*
 * Kernel timing over a measured region (no reference counterpart).  While
 * enabled, every launch made by the entry points above is bracketed by a pair
 * of HIP events on its stream.  sft_prof_collect() waits for the recorded
 * events, adds each launch's duration into total_ms[kind] / launches[kind]
 * (arrays of n_kinds entries, kinds numbered as sft_prof_kind_name) and forgets
 * them.  Enabling or disabling also forgets pending events.
 */
int sft_prof_enable(int on);
int sft_prof_num_kinds(void);
const char *sft_prof_kind_name(int kind);
int sft_prof_collect(double *total_ms, int64_t *launches, int n_kinds);

#ifdef __cplusplus
}
#endif

#endif /* SFT_FT_H */
