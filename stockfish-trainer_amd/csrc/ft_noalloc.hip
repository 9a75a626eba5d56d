// Allocation-free int16 forward (sft_ft_fwd_i16_noalloc) for callers that
// cannot allocate device memory: code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc.  Built alone into
// libsft_ft_noalloc.so, which links libsft_ft.so for the kernels, so that only
// the processes that load it reserve the scratch array below.
//
// It computes exactly what sft_ft_fwd_i16_ex computes with a workspace of
// sft_ft_fwd_i16_workspace_size() bytes: the table and its PSQT columns are
// packed into 64-column tiles and gathered XCD by XCD.  The packed tiles live
// in `scratch`, a file-scope device array of kScratchBytes that every GPU the
// library runs on holds until the process ends.  The host never names the
// array when it needs its memory: at the first call on a device (that device
// current) hipGetSymbolAddress gives that device's copy's address, which is
// kept per device and passed to the kernels like any workspace pointer.
//
// Every call on one GPU shares that GPU's array and leaves the last call's
// packed table in it.  The pack kernel writes every 16-byte chunk the gather
// reads (the padding lanes of the last tile are neither written nor read), so
// nothing needs clearing between calls.  Calls that overlap on one GPU (other
// host threads, other streams) race on the array; callers serialise them.
#include <mutex>

#include "common.h"
#include "sft_ft_noalloc.h"

namespace sft {

size_t fwd_i16_tiled_workspace(int64_t N, int L, int P);
bool fwd_i16_tiled_supported(int64_t N, int L, int P, const void *W, const void *bias, const void *out);
int i16_pack(const int16_t *W, int64_t N, int L, const int32_t *psqt, int P, void *packed, size_t bytes,
             hipStream_t s, const char *who);
int fwd_i16_packed(const int32_t *idx0, const int32_t *idx1, int64_t B, int K, const void *packed, int64_t N, int L,
                   const int16_t *bias, int P, int16_t *out0, int16_t *out1, int32_t *psqt_out0, int32_t *psqt_out1,
                   int lo, int hi, int wrap16, hipStream_t s, const char *who);
int fwd_i16(const int32_t *idx, int64_t B, int K, const int16_t *W, int64_t N, int L, const int16_t *bias,
            const int32_t *psqt, int P, int16_t *out, int32_t *psqt_out, int lo, int hi, int wrap16, hipStream_t s);
int check_i16_args(const char *who, const int32_t *idx, int64_t batch, int32_t max_active, const int16_t *weight,
                   int64_t num_inputs, int32_t output_size, const int16_t *bias, const int32_t *psqt_weight,
                   int32_t psqt_size, int16_t *out, int32_t *psqt_out, int32_t clip_lo, int32_t clip_hi,
                   uint32_t flags);

namespace {

constexpr size_t kScratchBytes = SFT_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes % 256 == 0, "the packed table starts 256-byte aligned");

__device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch[kMaxDevices];  // this device's copy of `scratch`, once looked up

// Address of the current device's copy of `scratch`, looked up once per device.
int scratch_on_current_device(void **ptr, const char *who) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(SFT_EHIP, std::string(who) + ": hipGetDevice: " + hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(SFT_EUNSUPPORTED, std::string(who) + ": device ordinal beyond 63");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(SFT_EHIP, std::string(who) + ": hipGetSymbolAddress(scratch): " + hipGetErrorString(e));
    if ((uintptr_t)p % 256 != 0) return fail(SFT_EHIP, std::string(who) + ": scratch is not 256-byte aligned");
    g_scratch[dev] = p;
  }
  *ptr = g_scratch[dev];
  return SFT_OK;
}

}  // namespace
}  // namespace sft

using namespace sft;

extern "C" int sft_ft_fwd_i16_noalloc(const int32_t *idx, int64_t batch, int32_t max_active, const int16_t *weight,
                                      int64_t num_inputs, int32_t output_size, const int16_t *bias,
                                      const int32_t *psqt_weight, int32_t psqt_size, int16_t *out,
                                      int32_t *psqt_out, int32_t clip_lo, int32_t clip_hi, uint32_t flags,
                                      void *stream) {
  const char *who = "sft_ft_fwd_i16_noalloc";
  clear_error();
  int rc = check_i16_args(who, idx, batch, max_active, weight, num_inputs, output_size, bias, psqt_weight, psqt_size,
                          out, psqt_out, clip_lo, clip_hi, flags);
  if (rc != SFT_OK) return rc;
  if (batch == 0) return SFT_OK;
  const int P = psqt_weight ? psqt_size : 0;
  const int wrap = (flags & SFT_Q16_WRAP16) ? 1 : 0;
  const hipStream_t s = (hipStream_t)stream;
  if ((flags & SFT_Q16_ROWS) || !fwd_i16_tiled_supported(num_inputs, output_size, P, weight, bias, out))
    return fwd_i16(idx, batch, max_active, weight, num_inputs, output_size, bias, psqt_weight, P, out, psqt_out,
                   clip_lo, clip_hi, wrap, s);  // the row gather uses no scratch
  const size_t need = fwd_i16_tiled_workspace(num_inputs, output_size, P);
  if (need > kScratchBytes)
    return fail(SFT_EWORKSPACE, std::string(who) + ": the packed table takes " + std::to_string(need) +
                                    " bytes, more than the " + std::to_string(kScratchBytes) +
                                    "-byte static scratch (SFT_NOALLOC_SCRATCH_BYTES); use sft_ft_fwd_i16_ex");
  void *ptr = nullptr;
  if ((rc = scratch_on_current_device(&ptr, who)) != SFT_OK) return rc;
  if ((rc = i16_pack(weight, num_inputs, output_size, psqt_weight, P, ptr, kScratchBytes, s, who)) != SFT_OK) return rc;
  return fwd_i16_packed(idx, nullptr, batch, max_active, ptr, num_inputs, output_size, bias, P, out, nullptr, psqt_out,
                        nullptr, clip_lo, clip_hi, wrap, s, who);
}
