/*
 * sft_ft_noalloc.h -- C ABI of libsft_ft_noalloc.so: the int16 quantized
 * forward for callers that cannot allocate device memory.
 *
 * No reference counterpart: it is for callers that cannot allocate (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc).  It lives
 * in a library of its own, linked against libsft_ft.so (which holds the
 * kernels, sft_last_error() and the conventions of sft_ft.h), because its
 * scratch is a static device array: each process that loads this library
 * reserves SFT_NOALLOC_SCRATCH_BYTES on every GPU it runs on, until the
 * process ends.  Processes that only load libsft_ft.so (training) reserve
 * nothing.
 */
#ifndef SFT_FT_NOALLOC_H
#define SFT_FT_NOALLOC_H

#include "sft_ft.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * int16 forward that allocates nothing and takes no workspace.  Same
 * arguments, flags and results, bit for bit, as sft_ft_fwd_i16_ex with a
 * workspace of sft_ft_fwd_i16_workspace_size() bytes (it compacts the index
 * rows once per column tile, as sft_ft_fwd_i16_packed, instead of building rank
 * lists, so its scratch need does not grow with the batch).  The packed tiles
 * go to the static device array of SFT_NOALLOC_SCRATCH_BYTES; a tiled shape
 * whose packed table is larger returns SFT_EWORKSPACE and launches nothing
 * (shapes outside the tiled path run the row gather, which needs no scratch).
 * All calls on one GPU share its array: calls that overlap on one GPU (other
 * threads or streams) race; serialise them.  Errors: sft_last_error().
 */
#define SFT_NOALLOC_SCRATCH_BYTES (64u << 20)
int sft_ft_fwd_i16_noalloc(const int32_t *idx, int64_t batch, int32_t max_active,
                           const int16_t *weight, int64_t num_inputs, int32_t output_size,
                           const int16_t *bias, const int32_t *psqt_weight, int32_t psqt_size,
                           int16_t *out, int32_t *psqt_out, int32_t clip_lo, int32_t clip_hi,
                           uint32_t flags, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SFT_FT_NOALLOC_H */
