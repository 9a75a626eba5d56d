// C ABI entry points of libsft_ft.so: host-side validation, dispatch, error
// reporting and the optional per-launch event timing.
#include <atomic>
#include <climits>
#include <memory>
#include <mutex>
#include <vector>

#include "common.h"

namespace sft {

int fwd_f32(const int32_t *idx, int64_t B, int K, const float *W, int64_t N, int L, const float *bias, float *out,
            hipStream_t s);
int fwd_i16(const int32_t *idx, int64_t B, int K, const int16_t *W, int64_t N, int L, const int16_t *bias,
            const int32_t *psqt, int P, int16_t *out, int32_t *psqt_out, int lo, int hi, int wrap16, hipStream_t s);
int quantize_i16(const float *x, int64_t n, float scale, int16_t *out, hipStream_t s);
size_t fwd_tiled_workspace(int64_t B, int K, int64_t N, int L);
bool fwd_tiled_supported(int64_t N, int L, const void *W, const void *bias, const void *out);
int fwd_f32_tiled(const int32_t *idx, int64_t B, int K, const float *W, int64_t N, int L, const float *bias, float *out,
                  void *ws, size_t ws_bytes, hipStream_t s);
int bwd_workspace(int64_t B, int K, int64_t N, int L, uint32_t flags, size_t *bytes);
size_t fwd_i16_tiled_workspace(int64_t N, int L, int P);
size_t fwd_i16_ex_workspace(int64_t B, int K, int64_t N, int L, int P);
bool fwd_i16_tiled_supported(int64_t N, int L, int P, const void *W, const void *bias, const void *out);
int fwd_i16_tiled(const int32_t *idx, int64_t B, int K, const int16_t *W, int64_t N, int L, const int16_t *bias,
                  const int32_t *psqt, int P, int16_t *out, int32_t *psqt_out, int lo, int hi, int wrap16, void *ws,
                  size_t ws_bytes, hipStream_t s);
int i16_pack(const int16_t *W, int64_t N, int L, const int32_t *psqt, int P, void *packed, size_t bytes,
             hipStream_t s, const char *who);
int fwd_i16_packed(const int32_t *idx0, const int32_t *idx1, int64_t B, int K, const void *packed, int64_t N, int L,
                   const int16_t *bias, int P, int16_t *out0, int16_t *out1, int32_t *psqt_out0, int32_t *psqt_out1,
                   int lo, int hi, int wrap16, hipStream_t s, const char *who);
size_t fwd_i16_ranked_workspace(int64_t B, int K, int persp);
int fwd_i16_packed_ranked(const int32_t *idx0, const int32_t *idx1, int64_t B, int K, const void *packed, int64_t N,
                          int L, const int16_t *bias, int P, int16_t *out0, int16_t *out1, int32_t *psqt_out0,
                          int32_t *psqt_out1, int lo, int hi, int wrap16, void *ws, size_t ws_bytes, hipStream_t s,
                          const char *who);
int bwd_f32(const int32_t *idx, int64_t B, int K, const float *grad, int64_t N, int L, float *dW, float *db,
            void *ws, size_t ws_bytes, uint32_t flags, hipStream_t s, void *prep = nullptr, size_t prep_bytes = 0);
int bwd_prep_bytes(int64_t B, int K, int64_t N, int L, uint32_t flags, size_t *bytes);
int bwd_prepare(const int32_t *idx, int64_t B, int K, int64_t N, int L, uint32_t flags, void *prep,
                size_t prep_bytes, hipStream_t s);
size_t index_lds_bytes(int G, int K);
int fwd_pair_f32(const int32_t *idx0, const int32_t *idx1, int64_t B, int K, const FoldSrc &src, int64_t N, int L,
                 const float *bias, float *out0, float *out1, void *ws, size_t ws_bytes, hipStream_t s);
size_t bwd_pair_workspace(int64_t B, int K, int64_t N, int L);
int bwd_pair_f32(const int32_t *idx0, const int32_t *idx1, int64_t B, int K, const float *grad0, const float *grad1,
                 int64_t N, int L, const RowDst &dst, const float *const *vgrad_src, float *const *vgrad,
                 const int64_t *vperiod, const int64_t *vreps, int nvirt, float *db, void *ws, size_t ws_bytes,
                 hipStream_t s);
void zero_f32(float *p, int64_t n, hipStream_t s);
int ranger_update_f32(float *p, const float *grad, float *variance_ma, float *gma_cur, const float *gma_prev,
                      int64_t rows, int64_t cols, const float *scalars, hipStream_t s);
size_t leb128_workspace(int64_t n);
int leb128_encode(const void *values, int elem, int64_t n, uint8_t *out, int64_t *out_len, void *ws, hipStream_t s);
int probe_l2_gather(const float *table, int64_t table_rows, int rounds, int blocks, float *out, hipStream_t s);
int encode_features(const uint8_t *boards, const uint8_t *stm, int64_t B, const int32_t *comps, int ncomp,
                    int32_t *white, int32_t *black, int K, float *us, int64_t *psqt, int64_t *ls, int32_t *count_w,
                    int32_t *count_b, hipStream_t s);
size_t map_tiles_workspace(const ColMap &m, int64_t rows);
size_t table_tiles_workspace(const ColMap &m, int64_t N);
size_t fwd_pair_workspace(const ColMap &m, int64_t B, int K, int64_t N, bool carry);
int fwd_transform_f32(const int32_t *idx0, const int32_t *idx1, int64_t B, int K, const FoldSrc &src, int64_t N,
                      int L, int L1, const float *bias, const float *us, const int64_t *psqt_idx, float *l0,
                      float *psqt, void *saved, size_t saved_bytes, void *ws, size_t ws_bytes, hipStream_t s);
size_t bwd_transform_workspace(int64_t B, int K, int64_t N, int L, int L1);
int bwd_transform_f32(const int32_t *idx0, const int32_t *idx1, int64_t B, int K, const float *g_l0,
                      const float *g_psqt, const float *us, const int64_t *psqt_idx, const void *saved,
                      size_t saved_bytes, int64_t N, int L, int L1, const RowDst &dst, const float *const *vgrad_src,
                      float *const *vgrad, const int64_t *vperiod, const int64_t *vreps, int nvirt, float *db,
                      void *ws, size_t ws_bytes, hipStream_t s);

namespace {
thread_local std::string t_error;
}

const char *error_cstr() { return t_error.c_str(); }
void set_error(const std::string &msg) { t_error = msg; }
void clear_error() { t_error.clear(); }
int fail(int code, const std::string &msg) {
  t_error = msg;
  return code;
}
int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SFT_EHIP, std::string(what) + ": " + hipGetErrorString(e));
  return SFT_OK;
}

// ------------------------------------------------------- side stream ----
// One non-blocking stream (default priority), a fork event and kSideMarks
// join events per thread and device, created on first use and kept until the
// thread ends: a call forks independent work onto the side stream and makes
// its own stream wait for marks recorded there before the work that needs it.
// Per thread, so that concurrent callers (and a caller capturing a graph)
// never share one.
namespace {
struct SideState {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr;
  hipEvent_t mark[kSideMarks] = {};
  ~SideState() {
    for (hipEvent_t &e : mark)
      if (e) (void)hipEventDestroy(e);
    if (fork) (void)hipEventDestroy(fork);
    if (stream) (void)hipStreamDestroy(stream);
  }
};
thread_local std::vector<std::unique_ptr<SideState>> t_side;

SideState *side_state(bool create) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  if ((int)t_side.size() <= dev) {
    if (!create) return nullptr;
    t_side.resize(dev + 1);
  }
  if (!t_side[dev] && create) {
    auto st = std::make_unique<SideState>();
    bool ok = hipStreamCreateWithFlags(&st->stream, hipStreamNonBlocking) == hipSuccess &&
              hipEventCreateWithFlags(&st->fork, hipEventDisableTiming) == hipSuccess;
    for (hipEvent_t &e : st->mark) ok = ok && hipEventCreateWithFlags(&e, hipEventDisableTiming) == hipSuccess;
    if (!ok) return nullptr;
    t_side[dev] = std::move(st);
  }
  return t_side[dev].get();
}
}  // namespace

int fork_side(hipStream_t s, hipStream_t *side) {
  SideState *st = side_state(true);
  if (!st) return fail(SFT_EHIP, "side stream: creation failed");
  if (hipEventRecord(st->fork, s) != hipSuccess || hipStreamWaitEvent(st->stream, st->fork, 0) != hipSuccess)
    return fail(SFT_EHIP, "side stream: fork failed");
  *side = st->stream;
  return SFT_OK;
}

int mark_side(int slot) {
  SideState *st = side_state(false);
  if (!st || slot < 0 || slot >= kSideMarks) return fail(SFT_EHIP, "side stream: mark without fork");
  if (hipEventRecord(st->mark[slot], st->stream) != hipSuccess) return fail(SFT_EHIP, "side stream: mark failed");
  return SFT_OK;
}

int wait_side(hipStream_t s, int slot) {
  SideState *st = side_state(false);
  if (!st || slot < 0 || slot >= kSideMarks) return fail(SFT_EHIP, "side stream: wait without fork");
  if (hipStreamWaitEvent(s, st->mark[slot], 0) != hipSuccess) return fail(SFT_EHIP, "side stream: wait failed");
  return SFT_OK;
}

int join_side(hipStream_t s) {
  const int rc = mark_side(0);
  return rc != SFT_OK ? rc : wait_side(s, 0);
}

SideJoinGuard::~SideJoinGuard() {
  if (!armed_) return;
  const std::string keep = t_error;
  (void)join_side(s_);
  t_error = keep;
}

Mapping choose_mapping(int64_t chunks, int min_group) {
  // Largest lane group whose single-slab lane use is >= 75%; otherwise the
  // single-slab mapping with the best lane use; rows too wide for one slab
  // use G = 64 and as few slabs as possible.
  static const int groups[4] = {64, 32, 16, 8};
  Mapping best{64, kMaxCpl, (int)ceil_div(chunks, (int64_t)kWave * kMaxCpl)};
  if (chunks > (int64_t)kWave * kMaxCpl) {
    best.cpl = (int)ceil_div(chunks, (int64_t)kWave * best.slabs);
    return best;
  }
  double best_eff = -1.0;
  for (int G : groups) {
    if (G < min_group) continue;
    const int64_t cpl = ceil_div(chunks, G);
    if (cpl > kMaxCpl) continue;
    const double eff = (double)chunks / (double)(G * cpl);
    if (eff >= 0.75) return Mapping{G, (int)cpl, 1};
    if (eff > best_eff) {
      best_eff = eff;
      best = Mapping{G, (int)cpl, 1};
    }
  }
  return best;
}

// ------------------------------------------------------------ profiling ----
namespace {
struct PendingLaunch {
  hipEvent_t start, stop;
  int kind;
};
std::atomic<bool> g_prof_on{false};
std::mutex g_prof_mu;
std::vector<PendingLaunch> g_pending;
std::vector<hipEvent_t> g_event_pool;

hipEvent_t take_event() {
  if (!g_event_pool.empty()) {
    hipEvent_t e = g_event_pool.back();
    g_event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

void drop_pending_locked() {
  for (auto &p : g_pending) {
    g_event_pool.push_back(p.start);
    g_event_pool.push_back(p.stop);
  }
  g_pending.clear();
}

struct ActiveScope {
  hipEvent_t start, stop;
  int kind;
  hipStream_t stream;
};

const char *const kKindNames[] = {
    "fwd_f32_gather",   "bwd_feature_sort",  "bwd_segment_offsets", "bwd_feature_gather", "bwd_bias_partial",
    "bwd_bias_final",   "bwd_atomic_scatter", "bwd_zero_fill",      "fwd_i16_gather",     "quantize_i16",
    "fwd_tile_relayout", "fwd_f32_tiled_gather", "bwd_tiled_gather", "fwd_i16_tiled_gather",
    "fwd_fold_relayout", "bwd_virtual_reduce", "bwd_epilogue", "ranger22_update", "encode_features", "leb128_encode",
    "probe_l2_gather", "fwd_rank_lists",
};
static_assert(sizeof(kKindNames) / sizeof(kKindNames[0]) == kProfNumKinds, "one name per profiling kind");
}  // namespace

ProfScope::ProfScope(int kind, hipStream_t stream) : slot_(nullptr) {
  if (!g_prof_on.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lock(g_prof_mu);
  hipEvent_t a = take_event(), b = take_event();
  if (!a || !b) return;
  if (hipEventRecord(a, stream) != hipSuccess) return;
  slot_ = new ActiveScope{a, b, kind, stream};
}

ProfScope::~ProfScope() {
  if (!slot_) return;
  ActiveScope *sc = static_cast<ActiveScope *>(slot_);
  std::lock_guard<std::mutex> lock(g_prof_mu);
  if (hipEventRecord(sc->stop, sc->stream) == hipSuccess) g_pending.push_back(PendingLaunch{sc->start, sc->stop, sc->kind});
  delete sc;
}

}  // namespace sft

using namespace sft;

namespace {

bool bad_sizes(int64_t B, int32_t K, int64_t N, int32_t L, std::string &why) {
  if (B < 0) why = "batch must be >= 0";
  else if (K <= 0) why = "max_active must be > 0";
  else if (N <= 0 || N >= INT32_MAX) why = "num_inputs must be in [1, 2^31-1)";
  else if (L <= 0) why = "output_size must be > 0";
  else if (B * (int64_t)K >= INT32_MAX) why = "batch * max_active must be < 2^31-1";
  else if ((int64_t)N * L >= ((int64_t)1 << 40) || B * (int64_t)L >= ((int64_t)1 << 40)) why = "tensor too large";
  else return false;
  return true;
}

}  // namespace

namespace sft {
// Host-side validation shared by the int16 forward entry points.
int check_i16_args(const char *who, const int32_t *idx, int64_t batch, int32_t max_active, const int16_t *weight,
                   int64_t num_inputs, int32_t output_size, const int16_t *bias, const int32_t *psqt_weight,
                   int32_t psqt_size, int16_t *out, int32_t *psqt_out, int32_t clip_lo, int32_t clip_hi,
                   uint32_t flags) {
  std::string why;
  const std::string w(who);
  if (bad_sizes(batch, max_active, num_inputs, output_size, why)) return fail(SFT_EINVAL, w + ": " + why);
  if (max_active >= 65536) return fail(SFT_EINVAL, w + ": max_active must be < 65536");
  if (!weight || !bias || (batch > 0 && (!idx || !out))) return fail(SFT_EINVAL, w + ": null pointer");
  if ((psqt_weight == nullptr) != (psqt_out == nullptr))
    return fail(SFT_EINVAL, w + ": psqt_weight and psqt_out must both be set or both be NULL");
  if (psqt_weight && (psqt_size <= 0 || psqt_size > kWave)) return fail(SFT_EINVAL, w + ": psqt_size must be in [1, 64]");
  if (clip_lo > clip_hi || clip_lo < -32768 || clip_hi > 32767)
    return fail(SFT_EINVAL, w + ": need -32768 <= clip_lo <= clip_hi <= 32767");
  if (flags & ~(SFT_Q16_WRAP16 | SFT_Q16_ROWS)) return fail(SFT_EINVAL, w + ": unknown flags");
  return SFT_OK;
}
}  // namespace sft

extern "C" {

int sft_abi_version(void) { return SFT_ABI_VERSION; }

const char *sft_last_error(void) { return error_cstr(); }

int sft_ft_fwd_f32(const int32_t *idx, int64_t batch, int32_t max_active, const float *weight, int64_t num_inputs,
                   int32_t output_size, const float *bias, float *out, void *stream) {
  clear_error();
  std::string why;
  if (bad_sizes(batch, max_active, num_inputs, output_size, why)) return fail(SFT_EINVAL, "sft_ft_fwd_f32: " + why);
  if (!weight || !bias || (batch > 0 && (!idx || !out))) return fail(SFT_EINVAL, "sft_ft_fwd_f32: null pointer");
  if (batch == 0) return SFT_OK;
  return fwd_f32(idx, batch, max_active, weight, num_inputs, output_size, bias, out, (hipStream_t)stream);
}

int sft_ft_fwd_f32_workspace_size(int64_t batch, int32_t max_active, int64_t num_inputs, int32_t output_size,
                                  uint32_t flags, size_t *bytes) {
  clear_error();
  std::string why;
  if (!bytes) return fail(SFT_EINVAL, "sft_ft_fwd_f32_workspace_size: null pointer");
  if (bad_sizes(batch, max_active, num_inputs, output_size, why))
    return fail(SFT_EINVAL, "sft_ft_fwd_f32_workspace_size: " + why);
  if (flags & ~SFT_FWD_ROWS) return fail(SFT_EINVAL, "sft_ft_fwd_f32_workspace_size: unknown flags");
  const bool tiled = !(flags & SFT_FWD_ROWS) && fwd_tiled_supported(num_inputs, output_size, nullptr, nullptr, nullptr);
  *bytes = tiled ? fwd_tiled_workspace(batch, max_active, num_inputs, output_size) : 0;
  return SFT_OK;
}

int sft_ft_fwd_f32_ex(const int32_t *idx, int64_t batch, int32_t max_active, const float *weight, int64_t num_inputs,
                      int32_t output_size, const float *bias, float *out, void *workspace, size_t workspace_bytes,
                      uint32_t flags, void *stream) {
  clear_error();
  std::string why;
  if (bad_sizes(batch, max_active, num_inputs, output_size, why)) return fail(SFT_EINVAL, "sft_ft_fwd_f32_ex: " + why);
  if (!weight || !bias || (batch > 0 && (!idx || !out))) return fail(SFT_EINVAL, "sft_ft_fwd_f32_ex: null pointer");
  if (flags & ~SFT_FWD_ROWS) return fail(SFT_EINVAL, "sft_ft_fwd_f32_ex: unknown flags");
  if (batch == 0) return SFT_OK;
  const bool tiled = !(flags & SFT_FWD_ROWS) && fwd_tiled_supported(num_inputs, output_size, weight, bias, out) &&
                     workspace != nullptr &&
                     workspace_bytes >= fwd_tiled_workspace(batch, max_active, num_inputs, output_size);
  if (tiled)
    return fwd_f32_tiled(idx, batch, max_active, weight, num_inputs, output_size, bias, out, workspace,
                         workspace_bytes, (hipStream_t)stream);
  return fwd_f32(idx, batch, max_active, weight, num_inputs, output_size, bias, out, (hipStream_t)stream);
}

int sft_ft_bwd_f32_workspace_size(int64_t batch, int32_t max_active, int64_t num_inputs, int32_t output_size,
                                  uint32_t flags, size_t *bytes) {
  clear_error();
  std::string why;
  if (!bytes) return fail(SFT_EINVAL, "sft_ft_bwd_f32_workspace_size: null pointer");
  if (bad_sizes(batch, max_active, num_inputs, output_size, why))
    return fail(SFT_EINVAL, "sft_ft_bwd_f32_workspace_size: " + why);
  if (flags & ~(SFT_BWD_OVERWRITE | SFT_BWD_ATOMIC | SFT_BWD_ROWS | SFT_BWD_PREPARED))
    return fail(SFT_EINVAL, "sft_ft_bwd_f32_workspace_size: unknown flags");
  return bwd_workspace(batch, max_active, num_inputs, output_size, flags, bytes);
}

int sft_ft_bwd_f32_prep_size(int64_t batch, int32_t max_active, int64_t num_inputs, int32_t output_size,
                             uint32_t flags, size_t *bytes) {
  clear_error();
  std::string why;
  if (!bytes) return fail(SFT_EINVAL, "sft_ft_bwd_f32_prep_size: null pointer");
  if (bad_sizes(batch, max_active, num_inputs, output_size, why))
    return fail(SFT_EINVAL, "sft_ft_bwd_f32_prep_size: " + why);
  if (flags & ~(SFT_BWD_OVERWRITE | SFT_BWD_ATOMIC | SFT_BWD_ROWS | SFT_BWD_PREPARED))
    return fail(SFT_EINVAL, "sft_ft_bwd_f32_prep_size: unknown flags");
  return bwd_prep_bytes(batch, max_active, num_inputs, output_size, flags, bytes);
}

int sft_ft_fwd_f32_prep(const int32_t *idx, int64_t batch, int32_t max_active, const float *weight,
                        int64_t num_inputs, int32_t output_size, const float *bias, float *out, void *workspace,
                        size_t workspace_bytes, uint32_t flags, void *prep, size_t prep_bytes, uint32_t bwd_flags,
                        void *stream) {
  clear_error();
  std::string why;
  if (bad_sizes(batch, max_active, num_inputs, output_size, why)) return fail(SFT_EINVAL, "sft_ft_fwd_f32_prep: " + why);
  if (!weight || !bias || (batch > 0 && (!idx || !out))) return fail(SFT_EINVAL, "sft_ft_fwd_f32_prep: null pointer");
  if (flags & ~SFT_FWD_ROWS) return fail(SFT_EINVAL, "sft_ft_fwd_f32_prep: unknown flags");
  if (bwd_flags & ~(SFT_BWD_OVERWRITE | SFT_BWD_ATOMIC | SFT_BWD_ROWS | SFT_BWD_PREPARED))
    return fail(SFT_EINVAL, "sft_ft_fwd_f32_prep: unknown backward flags");
  if (batch == 0) return SFT_OK;
  size_t need = 0;
  bwd_prep_bytes(batch, max_active, num_inputs, output_size, bwd_flags, &need);
  if (need > 0 && (prep == nullptr || prep_bytes < need || (uintptr_t)prep % 256 != 0))
    return fail(SFT_EWORKSPACE, "sft_ft_fwd_f32_prep: prepared buffer smaller than sft_ft_bwd_f32_prep_size() "
                                "or not 256-byte aligned");
  // The backward's sort needs the indices only: it runs on the side stream
  // beside the forward's kernels and is joined before the call returns.
  const hipStream_t s = (hipStream_t)stream;
  if (need == 0)
    return sft_ft_fwd_f32_ex(idx, batch, max_active, weight, num_inputs, output_size, bias, out, workspace,
                             workspace_bytes, flags, stream);
  hipStream_t side;
  int rc = fork_side(s, &side);
  if (rc != SFT_OK) return rc;
  SideJoinGuard side_join(s);
  if ((rc = bwd_prepare(idx, batch, max_active, num_inputs, output_size, bwd_flags, prep, prep_bytes, side)) != SFT_OK)
    return rc;
  const bool tiled = !(flags & SFT_FWD_ROWS) && fwd_tiled_supported(num_inputs, output_size, weight, bias, out) &&
                     workspace != nullptr &&
                     workspace_bytes >= fwd_tiled_workspace(batch, max_active, num_inputs, output_size);
  rc = tiled ? fwd_f32_tiled(idx, batch, max_active, weight, num_inputs, output_size, bias, out, workspace,
                             workspace_bytes, s)
             : fwd_f32(idx, batch, max_active, weight, num_inputs, output_size, bias, out, s);
  if (rc != SFT_OK) return rc;
  side_join.release();
  return join_side(s);
}

int sft_ft_bwd_f32_prepared(const int32_t *idx, int64_t batch, int32_t max_active, const float *grad_out,
                            int64_t num_inputs, int32_t output_size, float *weight_grad, float *bias_grad,
                            void *prep, size_t prep_bytes, void *workspace, size_t workspace_bytes, uint32_t flags,
                            void *stream) {
  clear_error();
  std::string why;
  if (bad_sizes(batch, max_active, num_inputs, output_size, why))
    return fail(SFT_EINVAL, "sft_ft_bwd_f32_prepared: " + why);
  if (!weight_grad || !bias_grad || (batch > 0 && (!idx || !grad_out)))
    return fail(SFT_EINVAL, "sft_ft_bwd_f32_prepared: null pointer");
  if (flags & ~(SFT_BWD_OVERWRITE | SFT_BWD_ATOMIC | SFT_BWD_ROWS | SFT_BWD_PREPARED))
    return fail(SFT_EINVAL, "sft_ft_bwd_f32_prepared: unknown flags");
  return bwd_f32(idx, batch, max_active, grad_out, num_inputs, output_size, weight_grad, bias_grad, workspace,
                 workspace_bytes, flags | SFT_BWD_PREPARED, (hipStream_t)stream, prep, prep_bytes);
}

int sft_ft_bwd_f32(const int32_t *idx, int64_t batch, int32_t max_active, const float *grad_out, int64_t num_inputs,
                   int32_t output_size, float *weight_grad, float *bias_grad, void *workspace, size_t workspace_bytes,
                   uint32_t flags, void *stream) {
  clear_error();
  std::string why;
  if (bad_sizes(batch, max_active, num_inputs, output_size, why)) return fail(SFT_EINVAL, "sft_ft_bwd_f32: " + why);
  if (!weight_grad || !bias_grad || (batch > 0 && (!idx || !grad_out)))
    return fail(SFT_EINVAL, "sft_ft_bwd_f32: null pointer");
  if (flags & ~(SFT_BWD_OVERWRITE | SFT_BWD_ATOMIC | SFT_BWD_ROWS)) return fail(SFT_EINVAL, "sft_ft_bwd_f32: unknown flags");
  return bwd_f32(idx, batch, max_active, grad_out, num_inputs, output_size, weight_grad, bias_grad, workspace,
                 workspace_bytes, flags, (hipStream_t)stream);
}

// Validates the block description of a composed table and its shape; sets *N.
static int check_pair_shape(const char *who, int64_t batch, int32_t max_active, int32_t num_blocks,
                            const int64_t *block_rows, const int64_t *block_virtual_rows, int32_t output_size,
                            int64_t *N) {
  const std::string w(who);
  if (num_blocks < 1 || num_blocks > kMaxBlocks) return fail(SFT_EINVAL, w + ": num_blocks must be in [1, 4]");
  if (!block_rows || !block_virtual_rows) return fail(SFT_EINVAL, w + ": null pointer");
  int64_t n = 0;
  for (int s = 0; s < num_blocks; ++s) {
    const int64_t r = block_rows[s], v = block_virtual_rows[s];
    if (r <= 0 || r >= INT32_MAX) return fail(SFT_EINVAL, w + ": block_rows must be in [1, 2^31-1)");
    if (v < 0 || (v > 0 && r % v != 0))
      return fail(SFT_EINVAL, w + ": block_virtual_rows must be 0 or divide block_rows");
    n += r;
  }
  std::string why;
  if (bad_sizes(batch, max_active, n, output_size, why)) return fail(SFT_EINVAL, w + ": " + why);
  if (output_size % 4 != 0 || output_size < 256)
    return fail(SFT_EUNSUPPORTED, w + ": output_size must be a multiple of 4 and >= 256");
  if (!fwd_tiled_supported(n, output_size, nullptr, nullptr, nullptr) || n * (int64_t)(output_size / 4) >= INT32_MAX)
    return fail(SFT_EUNSUPPORTED, w + ": table too large for the tiled composed path");
  if (index_lds_bytes(8, max_active) > kMaxIndexLds)
    return fail(SFT_EUNSUPPORTED, w + ": max_active too large for the LDS index lists");
  if (batch * 128 > (int64_t)UINT32_MAX)  // grad tile rows are 32-bit offsets
    return fail(SFT_EUNSUPPORTED, w + ": batch above 2^25 for the tiled composed path");
  *N = n;
  return SFT_OK;
}

static bool misaligned16(const void *p) { return (uintptr_t)p % 16 != 0; }

int sft_ft_pair_workspace_size(int64_t batch, int32_t max_active, int32_t num_blocks, const int64_t *block_rows,
                               const int64_t *block_virtual_rows, int32_t output_size, size_t *fwd_bytes,
                               size_t *bwd_bytes) {
  clear_error();
  if (!fwd_bytes || !bwd_bytes) return fail(SFT_EINVAL, "sft_ft_pair_workspace_size: null pointer");
  int64_t N = 0;
  const int rc = check_pair_shape("sft_ft_pair_workspace_size", batch, max_active, num_blocks, block_rows,
                                  block_virtual_rows, output_size, &N);
  if (rc != SFT_OK) return rc;
  *fwd_bytes = fwd_pair_workspace(plain_map(output_size / 4), batch, max_active, N, true);
  *bwd_bytes = bwd_pair_workspace(batch, max_active, N, output_size);
  return SFT_OK;
}

int sft_ft_fwd_pair_f32(const int32_t *idx0, const int32_t *idx1, int64_t batch, int32_t max_active,
                        int32_t num_blocks, const float *const *block_weight, const float *const *block_virtual,
                        const int64_t *block_rows, const int64_t *block_virtual_rows, int32_t output_size,
                        const float *bias, float *out0, float *out1, void *workspace, size_t workspace_bytes,
                        void *stream) {
  clear_error();
  const char *who = "sft_ft_fwd_pair_f32";
  int64_t N = 0;
  int rc = check_pair_shape(who, batch, max_active, num_blocks, block_rows, block_virtual_rows, output_size, &N);
  if (rc != SFT_OK) return rc;
  if (!block_weight || !block_virtual || !bias || (batch > 0 && (!idx0 || !idx1 || !out0 || !out1)))
    return fail(SFT_EINVAL, std::string(who) + ": null pointer");
  FoldSrc src{};
  src.n = num_blocks;
  for (int s = 0; s < num_blocks; ++s) {
    if (!block_weight[s] || (block_virtual_rows[s] > 0 && !block_virtual[s]))
      return fail(SFT_EINVAL, std::string(who) + ": null block pointer");
    if (misaligned16(block_weight[s]) || (block_virtual_rows[s] > 0 && misaligned16(block_virtual[s])))
      return fail(SFT_EINVAL, std::string(who) + ": block tables must be 16-byte aligned");
    src.start[s + 1] = src.start[s] + block_rows[s];
    src.w[s] = reinterpret_cast<const f32x4 *>(block_weight[s]);
    src.v[s] = block_virtual_rows[s] > 0 ? reinterpret_cast<const f32x4 *>(block_virtual[s]) : nullptr;
    src.period[s] = block_virtual_rows[s] > 0 ? block_virtual_rows[s] : 1;
  }
  if (misaligned16(bias) || (batch > 0 && (misaligned16(out0) || misaligned16(out1))))
    return fail(SFT_EINVAL, std::string(who) + ": bias and outputs must be 16-byte aligned");
  if (batch == 0) return SFT_OK;
  return fwd_pair_f32(idx0, idx1, batch, max_active, src, N, output_size, bias, out0, out1, workspace,
                      workspace_bytes, (hipStream_t)stream);
}

int sft_ft_bwd_pair_f32(const int32_t *idx0, const int32_t *idx1, int64_t batch, int32_t max_active,
                        const float *grad0, const float *grad1, int32_t num_blocks, const int64_t *block_rows,
                        const int64_t *block_virtual_rows, int32_t output_size, float *const *block_weight_grad,
                        float *const *block_virtual_grad, float *bias_grad, void *workspace, size_t workspace_bytes,
                        void *stream) {
  clear_error();
  const char *who = "sft_ft_bwd_pair_f32";
  int64_t N = 0;
  int rc = check_pair_shape(who, batch, max_active, num_blocks, block_rows, block_virtual_rows, output_size, &N);
  if (rc != SFT_OK) return rc;
  if (!block_weight_grad || !block_virtual_grad || !bias_grad || (batch > 0 && (!idx0 || !idx1 || !grad0 || !grad1)))
    return fail(SFT_EINVAL, std::string(who) + ": null pointer");
  RowDst dst{};
  dst.n = num_blocks;
  const float *vsrc[kMaxBlocks];
  float *vdst[kMaxBlocks];
  int64_t vperiod[kMaxBlocks], vreps[kMaxBlocks];
  int nvirt = 0;
  for (int s = 0; s < num_blocks; ++s) {
    if (!block_weight_grad[s] || (block_virtual_rows[s] > 0 && !block_virtual_grad[s]))
      return fail(SFT_EINVAL, std::string(who) + ": null block pointer");
    if (misaligned16(block_weight_grad[s]) || (block_virtual_rows[s] > 0 && misaligned16(block_virtual_grad[s])))
      return fail(SFT_EINVAL, std::string(who) + ": block grads must be 16-byte aligned");
    dst.start[s + 1] = dst.start[s] + block_rows[s];
    dst.p[s] = reinterpret_cast<f32x4 *>(block_weight_grad[s]);
    if (block_virtual_rows[s] > 0) {
      vsrc[nvirt] = block_weight_grad[s];
      vdst[nvirt] = block_virtual_grad[s];
      vperiod[nvirt] = block_virtual_rows[s];
      vreps[nvirt] = block_rows[s] / block_virtual_rows[s];
      ++nvirt;
    }
  }
  if (misaligned16(bias_grad) || (batch > 0 && (misaligned16(grad0) || misaligned16(grad1))))
    return fail(SFT_EINVAL, std::string(who) + ": bias_grad and grads must be 16-byte aligned");
  const hipStream_t st = (hipStream_t)stream;
  if (batch == 0) {  // no positions: every grad is zero
    for (int s = 0; s < num_blocks; ++s) {
      zero_f32(block_weight_grad[s], block_rows[s] * output_size, st);
      if (block_virtual_rows[s] > 0) zero_f32(block_virtual_grad[s], block_virtual_rows[s] * output_size, st);
    }
    zero_f32(bias_grad, output_size, st);
    return check_launch("sft_ft_bwd_pair_f32 (zero fill)");
  }
  return bwd_pair_f32(idx0, idx1, batch, max_active, grad0, grad1, N, output_size, dst, vsrc, vdst, vperiod, vreps,
                      nvirt, bias_grad, workspace, workspace_bytes, st);
}

static int check_l1(const char *who, int32_t output_size, int32_t l1) {
  if (l1 <= 0 || l1 >= output_size || l1 % 8 != 0)
    return fail(SFT_EUNSUPPORTED, std::string(who) + ": l1 must be a positive multiple of 8 below output_size");
  return SFT_OK;
}

static int make_fold_src(const char *who, int32_t num_blocks, const float *const *block_weight,
                         const float *const *block_virtual, const int64_t *block_rows,
                         const int64_t *block_virtual_rows, FoldSrc &src) {
  if (!block_weight || !block_virtual) return fail(SFT_EINVAL, std::string(who) + ": null pointer");
  src = FoldSrc{};
  src.n = num_blocks;
  for (int s = 0; s < num_blocks; ++s) {
    if (!block_weight[s] || (block_virtual_rows[s] > 0 && !block_virtual[s]))
      return fail(SFT_EINVAL, std::string(who) + ": null block pointer");
    if (misaligned16(block_weight[s]) || (block_virtual_rows[s] > 0 && misaligned16(block_virtual[s])))
      return fail(SFT_EINVAL, std::string(who) + ": block tables must be 16-byte aligned");
    src.start[s + 1] = src.start[s] + block_rows[s];
    src.w[s] = reinterpret_cast<const f32x4 *>(block_weight[s]);
    src.v[s] = block_virtual_rows[s] > 0 ? reinterpret_cast<const f32x4 *>(block_virtual[s]) : nullptr;
    src.period[s] = block_virtual_rows[s] > 0 ? block_virtual_rows[s] : 1;
  }
  return SFT_OK;
}

struct GradDst {
  RowDst dst;
  const float *vsrc[kMaxBlocks];
  float *vdst[kMaxBlocks];
  int64_t vperiod[kMaxBlocks], vreps[kMaxBlocks];
  int nvirt;
};

static int make_grad_dst(const char *who, int32_t num_blocks, const int64_t *block_rows,
                         const int64_t *block_virtual_rows, float *const *block_weight_grad,
                         float *const *block_virtual_grad, GradDst &g) {
  if (!block_weight_grad || !block_virtual_grad) return fail(SFT_EINVAL, std::string(who) + ": null pointer");
  g = GradDst{};
  g.dst.n = num_blocks;
  for (int s = 0; s < num_blocks; ++s) {
    if (!block_weight_grad[s] || (block_virtual_rows[s] > 0 && !block_virtual_grad[s]))
      return fail(SFT_EINVAL, std::string(who) + ": null block pointer");
    if (misaligned16(block_weight_grad[s]) || (block_virtual_rows[s] > 0 && misaligned16(block_virtual_grad[s])))
      return fail(SFT_EINVAL, std::string(who) + ": block grads must be 16-byte aligned");
    g.dst.start[s + 1] = g.dst.start[s] + block_rows[s];
    g.dst.p[s] = reinterpret_cast<f32x4 *>(block_weight_grad[s]);
    if (block_virtual_rows[s] > 0) {
      g.vsrc[g.nvirt] = block_weight_grad[s];
      g.vdst[g.nvirt] = block_virtual_grad[s];
      g.vperiod[g.nvirt] = block_virtual_rows[s];
      g.vreps[g.nvirt] = block_rows[s] / block_virtual_rows[s];
      ++g.nvirt;
    }
  }
  return SFT_OK;
}

static int zero_grads(int32_t num_blocks, const int64_t *block_rows, const int64_t *block_virtual_rows,
                      int32_t output_size, float *const *block_weight_grad, float *const *block_virtual_grad,
                      float *bias_grad, hipStream_t st, const char *who) {
  for (int s = 0; s < num_blocks; ++s) {
    zero_f32(block_weight_grad[s], block_rows[s] * output_size, st);
    if (block_virtual_rows[s] > 0) zero_f32(block_virtual_grad[s], block_virtual_rows[s] * output_size, st);
  }
  zero_f32(bias_grad, output_size, st);
  return check_launch(who);
}

int sft_ft_transform_workspace_size(int64_t batch, int32_t max_active, int32_t num_blocks, const int64_t *block_rows,
                                    const int64_t *block_virtual_rows, int32_t output_size, int32_t l1,
                                    size_t *saved_bytes, size_t *fwd_bytes, size_t *bwd_bytes) {
  clear_error();
  const char *who = "sft_ft_transform_workspace_size";
  if (!saved_bytes || !fwd_bytes || !bwd_bytes) return fail(SFT_EINVAL, std::string(who) + ": null pointer");
  int64_t N = 0;
  int rc = check_pair_shape(who, batch, max_active, num_blocks, block_rows, block_virtual_rows, output_size, &N);
  if (rc != SFT_OK || (rc = check_l1(who, output_size, l1)) != SFT_OK) return rc;
  const ColMap map = paired_map(output_size / 4, l1 / 8);
  *saved_bytes = 2 * map_tiles_workspace(map, batch);
  *fwd_bytes = fwd_pair_workspace(map, batch, max_active, N, false);
  *bwd_bytes = bwd_transform_workspace(batch, max_active, N, output_size, l1);
  return SFT_OK;
}

int sft_ft_fwd_transform_f32(const int32_t *idx0, const int32_t *idx1, int64_t batch, int32_t max_active,
                             int32_t num_blocks, const float *const *block_weight, const float *const *block_virtual,
                             const int64_t *block_rows, const int64_t *block_virtual_rows, int32_t output_size,
                             int32_t l1, const float *bias, const float *us, const int64_t *psqt_indices, float *l0,
                             float *psqt, void *saved, size_t saved_bytes, void *workspace, size_t workspace_bytes,
                             void *stream) {
  clear_error();
  const char *who = "sft_ft_fwd_transform_f32";
  int64_t N = 0;
  int rc = check_pair_shape(who, batch, max_active, num_blocks, block_rows, block_virtual_rows, output_size, &N);
  if (rc != SFT_OK || (rc = check_l1(who, output_size, l1)) != SFT_OK) return rc;
  if (!bias || (batch > 0 && (!idx0 || !idx1 || !us || !psqt_indices || !l0 || !psqt)))
    return fail(SFT_EINVAL, std::string(who) + ": null pointer");
  FoldSrc src;
  if ((rc = make_fold_src(who, num_blocks, block_weight, block_virtual, block_rows, block_virtual_rows, src)) != SFT_OK)
    return rc;
  if (misaligned16(bias) || (batch > 0 && misaligned16(l0)))
    return fail(SFT_EINVAL, std::string(who) + ": bias and l0 must be 16-byte aligned");
  if (batch == 0) return SFT_OK;
  return fwd_transform_f32(idx0, idx1, batch, max_active, src, N, output_size, l1, bias, us, psqt_indices, l0, psqt,
                           saved, saved_bytes, workspace, workspace_bytes, (hipStream_t)stream);
}

int sft_ft_bwd_transform_f32(const int32_t *idx0, const int32_t *idx1, int64_t batch, int32_t max_active,
                             const float *grad_l0, const float *grad_psqt, const float *us,
                             const int64_t *psqt_indices, const void *saved, size_t saved_bytes, int32_t num_blocks,
                             const int64_t *block_rows, const int64_t *block_virtual_rows, int32_t output_size,
                             int32_t l1, float *const *block_weight_grad, float *const *block_virtual_grad,
                             float *bias_grad, void *workspace, size_t workspace_bytes, void *stream) {
  clear_error();
  const char *who = "sft_ft_bwd_transform_f32";
  int64_t N = 0;
  int rc = check_pair_shape(who, batch, max_active, num_blocks, block_rows, block_virtual_rows, output_size, &N);
  if (rc != SFT_OK || (rc = check_l1(who, output_size, l1)) != SFT_OK) return rc;
  if (!bias_grad || (batch > 0 && (!idx0 || !idx1 || !grad_l0 || !grad_psqt || !us || !psqt_indices)))
    return fail(SFT_EINVAL, std::string(who) + ": null pointer");
  GradDst g;
  if ((rc = make_grad_dst(who, num_blocks, block_rows, block_virtual_rows, block_weight_grad, block_virtual_grad,
                          g)) != SFT_OK)
    return rc;
  if (misaligned16(bias_grad) || (batch > 0 && misaligned16(grad_l0)))
    return fail(SFT_EINVAL, std::string(who) + ": bias_grad and grad_l0 must be 16-byte aligned");
  const hipStream_t st = (hipStream_t)stream;
  if (batch == 0)
    return zero_grads(num_blocks, block_rows, block_virtual_rows, output_size, block_weight_grad, block_virtual_grad,
                      bias_grad, st, who);
  return bwd_transform_f32(idx0, idx1, batch, max_active, grad_l0, grad_psqt, us, psqt_indices, saved, saved_bytes, N,
                           output_size, l1, g.dst, g.vsrc, g.vdst, g.vperiod, g.vreps, g.nvirt, bias_grad, workspace,
                           workspace_bytes, st);
}

int sft_ranger22_update_f32(float *p, const float *grad, float *variance_ma, float *grad_ma_cur,
                            const float *grad_ma_prev, int64_t rows, int64_t cols, const float *scalars,
                            void *stream) {
  clear_error();
  if (!p || !grad || !variance_ma || !grad_ma_cur || !grad_ma_prev || !scalars)
    return fail(SFT_EINVAL, "sft_ranger22_update_f32: null pointer");
  if (rows < 0 || cols <= 0 || rows >= INT32_MAX || rows * cols >= ((int64_t)1 << 40))
    return fail(SFT_EINVAL, "sft_ranger22_update_f32: rows must be in [0, 2^31-1), cols > 0");
  if (rows == 0) return SFT_OK;
  return ranger_update_f32(p, grad, variance_ma, grad_ma_cur, grad_ma_prev, rows, cols, scalars, (hipStream_t)stream);
}

int sft_encode_features(const uint8_t *boards, const uint8_t *side_to_move, int64_t batch, const int32_t *components,
                        int32_t num_components, int32_t *white_indices, int32_t *black_indices, int32_t max_active,
                        float *us, int64_t *psqt_indices, int64_t *layer_stack_indices, int32_t *white_count,
                        int32_t *black_count, void *stream) {
  clear_error();
  const char *who = "sft_encode_features";
  if (batch < 0 || batch >= ((int64_t)1 << 30)) return fail(SFT_EINVAL, std::string(who) + ": batch out of range");
  if (!components || num_components < 1 || num_components > 2)
    return fail(SFT_EINVAL, std::string(who) + ": 1 or 2 components");
  int K = 0;
  for (int i = 0; i < num_components; ++i) {
    if (components[i] != SFT_FEATURES_THREATS && components[i] != SFT_FEATURES_HALFKA)
      return fail(SFT_EINVAL, std::string(who) + ": unknown component");
    if (i > 0 && components[i] == components[0]) return fail(SFT_EINVAL, std::string(who) + ": repeated component");
    K += components[i] == SFT_FEATURES_THREATS ? 128 : 32;
  }
  if (max_active != K) return fail(SFT_EINVAL, std::string(who) + ": max_active must be the components' sum");
  if (batch == 0) return SFT_OK;
  if (!boards || !side_to_move || !white_indices || !black_indices)
    return fail(SFT_EINVAL, std::string(who) + ": null pointer");
  if (misaligned16(boards) || misaligned16(white_indices) || misaligned16(black_indices))
    return fail(SFT_EINVAL, std::string(who) + ": boards and index rows must be 16-byte aligned");
  return encode_features(boards, side_to_move, batch, components, num_components, white_indices, black_indices, K, us,
                         psqt_indices, layer_stack_indices, white_count, black_count, (hipStream_t)stream);
}

int sft_leb128_workspace_size(int64_t n, size_t *bytes) {
  clear_error();
  if (!bytes) return fail(SFT_EINVAL, "sft_leb128_workspace_size: null pointer");
  if (n < 0 || n >= ((int64_t)1 << 40)) return fail(SFT_EINVAL, "sft_leb128_workspace_size: n out of range");
  *bytes = leb128_workspace(n);
  return SFT_OK;
}

int sft_leb128_encode(const void *values, int32_t elem_bytes, int64_t n, uint8_t *out, size_t out_capacity,
                      int64_t *out_len, void *workspace, size_t workspace_bytes, void *stream) {
  clear_error();
  const char *who = "sft_leb128_encode";
  if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4)
    return fail(SFT_EINVAL, std::string(who) + ": elem_bytes must be 1, 2 or 4");
  if (n < 0 || n >= ((int64_t)1 << 40)) return fail(SFT_EINVAL, std::string(who) + ": n out of range");
  if (!out_len || (n > 0 && (!values || !out))) return fail(SFT_EINVAL, std::string(who) + ": null pointer");
  const int64_t max_bytes = elem_bytes == 1 ? 2 : elem_bytes == 2 ? 3 : 5;  // signed LEB128 of 8/16/32-bit values
  if ((int64_t)out_capacity < n * max_bytes)
    return fail(SFT_EINVAL, std::string(who) + ": out_capacity must be at least n * (2, 3 or 5)");
  if (!workspace || workspace_bytes < leb128_workspace(n) || (uintptr_t)workspace % 8 != 0)
    return fail(SFT_EWORKSPACE, std::string(who) + ": workspace smaller than sft_leb128_workspace_size()");
  if ((uintptr_t)values % elem_bytes != 0 || (uintptr_t)out_len % 8 != 0)
    return fail(SFT_EINVAL, std::string(who) + ": misaligned values or out_len");
  return leb128_encode(values, elem_bytes, n, out, out_len, workspace, (hipStream_t)stream);
}


int sft_ft_fwd_i16(const int32_t *idx, int64_t batch, int32_t max_active, const int16_t *weight, int64_t num_inputs,
                   int32_t output_size, const int16_t *bias, const int32_t *psqt_weight, int32_t psqt_size,
                   int16_t *out, int32_t *psqt_out, int32_t clip_lo, int32_t clip_hi, uint32_t flags, void *stream) {
  clear_error();
  int rc = check_i16_args("sft_ft_fwd_i16", idx, batch, max_active, weight, num_inputs, output_size, bias, psqt_weight,
                          psqt_size, out, psqt_out, clip_lo, clip_hi, flags);
  if (rc != SFT_OK) return rc;
  if (batch == 0) return SFT_OK;
  return fwd_i16(idx, batch, max_active, weight, num_inputs, output_size, bias, psqt_weight,
                 psqt_weight ? psqt_size : 0, out, psqt_out, clip_lo, clip_hi, (flags & SFT_Q16_WRAP16) ? 1 : 0,
                 (hipStream_t)stream);
}

int sft_ft_fwd_i16_workspace_size(int64_t batch, int32_t max_active, int64_t num_inputs, int32_t output_size,
                                  int32_t psqt_size, uint32_t flags, size_t *bytes) {
  clear_error();
  std::string why;
  if (!bytes) return fail(SFT_EINVAL, "sft_ft_fwd_i16_workspace_size: null pointer");
  if (bad_sizes(batch, max_active, num_inputs, output_size, why))
    return fail(SFT_EINVAL, "sft_ft_fwd_i16_workspace_size: " + why);
  if (flags & ~(SFT_Q16_WRAP16 | SFT_Q16_ROWS)) return fail(SFT_EINVAL, "sft_ft_fwd_i16_workspace_size: unknown flags");
  const bool tiled = !(flags & SFT_Q16_ROWS) &&
                     fwd_i16_tiled_supported(num_inputs, output_size, psqt_size, nullptr, nullptr, nullptr);
  *bytes = tiled ? fwd_i16_ex_workspace(batch, max_active, num_inputs, output_size, psqt_size) : 0;
  return SFT_OK;
}

int sft_ft_fwd_i16_ex(const int32_t *idx, int64_t batch, int32_t max_active, const int16_t *weight,
                      int64_t num_inputs, int32_t output_size, const int16_t *bias, const int32_t *psqt_weight,
                      int32_t psqt_size, int16_t *out, int32_t *psqt_out, int32_t clip_lo, int32_t clip_hi,
                      void *workspace, size_t workspace_bytes, uint32_t flags, void *stream) {
  clear_error();
  int rc = check_i16_args("sft_ft_fwd_i16_ex", idx, batch, max_active, weight, num_inputs, output_size, bias,
                          psqt_weight, psqt_size, out, psqt_out, clip_lo, clip_hi, flags);
  if (rc != SFT_OK) return rc;
  if (batch == 0) return SFT_OK;
  const int P = psqt_weight ? psqt_size : 0;
  const int wrap = (flags & SFT_Q16_WRAP16) ? 1 : 0;
  const bool tiled = !(flags & SFT_Q16_ROWS) && fwd_i16_tiled_supported(num_inputs, output_size, P, weight, bias, out) &&
                     workspace != nullptr &&
                     workspace_bytes >= fwd_i16_ex_workspace(batch, max_active, num_inputs, output_size, P);
  if (tiled)
    return fwd_i16_tiled(idx, batch, max_active, weight, num_inputs, output_size, bias, psqt_weight, P, out, psqt_out,
                         clip_lo, clip_hi, wrap, workspace, workspace_bytes, (hipStream_t)stream);
  return fwd_i16(idx, batch, max_active, weight, num_inputs, output_size, bias, psqt_weight, P, out, psqt_out, clip_lo,
                 clip_hi, wrap, (hipStream_t)stream);
}

int sft_ft_i16_packed_size(int64_t num_inputs, int32_t output_size, int32_t psqt_size, size_t *bytes) {
  clear_error();
  std::string why;
  if (!bytes) return fail(SFT_EINVAL, "sft_ft_i16_packed_size: null pointer");
  if (bad_sizes(0, 1, num_inputs, output_size, why)) return fail(SFT_EINVAL, "sft_ft_i16_packed_size: " + why);
  if (psqt_size < 0) return fail(SFT_EINVAL, "sft_ft_i16_packed_size: psqt_size must be >= 0");
  if (!fwd_i16_tiled_supported(num_inputs, output_size, psqt_size, nullptr, nullptr, nullptr))
    return fail(SFT_EUNSUPPORTED, "sft_ft_i16_packed_size: needs output_size % 8 == 0, at least 8 tiles of 64 "
                                  "columns, psqt_size <= 8 and num_inputs * 128 <= 64 MiB");
  *bytes = fwd_i16_tiled_workspace(num_inputs, output_size, psqt_size);
  return SFT_OK;
}

int sft_ft_i16_pack(const int16_t *weight, int64_t num_inputs, int32_t output_size, const int32_t *psqt_weight,
                    int32_t psqt_size, void *packed, size_t packed_bytes, void *stream) {
  clear_error();
  std::string why;
  if (bad_sizes(0, 1, num_inputs, output_size, why)) return fail(SFT_EINVAL, "sft_ft_i16_pack: " + why);
  if (!weight || !packed) return fail(SFT_EINVAL, "sft_ft_i16_pack: null pointer");
  if ((psqt_weight == nullptr) != (psqt_size == 0))
    return fail(SFT_EINVAL, "sft_ft_i16_pack: psqt_size must be 0 exactly when psqt_weight is NULL");
  if (psqt_size < 0 || !fwd_i16_tiled_supported(num_inputs, output_size, psqt_size, weight, nullptr, nullptr))
    return fail(SFT_EUNSUPPORTED, "sft_ft_i16_pack: shape outside the tiled path (see sft_ft_i16_packed_size) "
                                  "or weight not 16-byte aligned");
  return i16_pack(weight, num_inputs, output_size, psqt_weight, psqt_size, packed, packed_bytes, (hipStream_t)stream,
                  "sft_ft_i16_pack");
}

// The checks both packed-table forwards make before anything runs.
static int check_i16_packed_call(const char *w, const int32_t *idx0, const int32_t *idx1, int64_t batch,
                                 int32_t max_active, const void *packed, size_t packed_bytes, int64_t num_inputs,
                                 int32_t output_size, const int16_t *bias, int32_t psqt_size, int16_t *out0,
                                 int16_t *out1, int32_t *psqt_out0, int32_t *psqt_out1, int32_t clip_lo,
                                 int32_t clip_hi, uint32_t flags) {
  std::string why;
  if (bad_sizes(batch, max_active, num_inputs, output_size, why)) return fail(SFT_EINVAL, std::string(w) + ": " + why);
  if (max_active >= 65536) return fail(SFT_EINVAL, std::string(w) + ": max_active must be < 65536");
  if (!packed || !bias) return fail(SFT_EINVAL, std::string(w) + ": null pointer");
  if (batch > 0 && (!idx0 || !out0 || (idx1 && !out1)))
    return fail(SFT_EINVAL, std::string(w) + ": null pointer");
  if (psqt_size < 0 || (batch > 0 && psqt_size > 0 && (!psqt_out0 || (idx1 && !psqt_out1))))
    return fail(SFT_EINVAL, std::string(w) + ": psqt outputs must be set when psqt_size > 0");
  if (clip_lo > clip_hi || clip_lo < -32768 || clip_hi > 32767)
    return fail(SFT_EINVAL, std::string(w) + ": need -32768 <= clip_lo <= clip_hi <= 32767");
  if (flags & ~SFT_Q16_WRAP16) return fail(SFT_EINVAL, std::string(w) + ": unknown flags");
  if ((uintptr_t)packed % 256 != 0 ||
      !fwd_i16_tiled_supported(num_inputs, output_size, psqt_size, bias, out0, idx1 ? out1 : out0))
    return fail(SFT_EUNSUPPORTED, std::string(w) + ": shape outside the tiled path, packed not 256-byte aligned, "
                                                   "or bias / outputs not 16-byte aligned");
  if (packed_bytes < fwd_i16_tiled_workspace(num_inputs, output_size, psqt_size))
    return fail(SFT_EINVAL, std::string(w) + ": packed_bytes smaller than sft_ft_i16_packed_size() for these sizes");
  return SFT_OK;
}

int sft_ft_fwd_i16_packed(const int32_t *idx0, const int32_t *idx1, int64_t batch, int32_t max_active,
                          const void *packed, size_t packed_bytes, int64_t num_inputs, int32_t output_size,
                          const int16_t *bias,
                          int32_t psqt_size, int16_t *out0, int16_t *out1, int32_t *psqt_out0, int32_t *psqt_out1,
                          int32_t clip_lo, int32_t clip_hi, uint32_t flags, void *stream) {
  clear_error();
  const char *w = "sft_ft_fwd_i16_packed";
  const int rc = check_i16_packed_call(w, idx0, idx1, batch, max_active, packed, packed_bytes, num_inputs, output_size,
                                       bias, psqt_size, out0, out1, psqt_out0, psqt_out1, clip_lo, clip_hi, flags);
  if (rc != SFT_OK) return rc;
  return fwd_i16_packed(idx0, idx1, batch, max_active, packed, num_inputs, output_size, bias, psqt_size, out0, out1,
                        psqt_size > 0 ? psqt_out0 : nullptr, psqt_size > 0 ? psqt_out1 : nullptr, clip_lo, clip_hi,
                        (flags & SFT_Q16_WRAP16) ? 1 : 0, (hipStream_t)stream, w);
}

int sft_ft_fwd_i16_packed_workspace_size(int64_t batch, int32_t max_active, int32_t perspectives, size_t *bytes) {
  clear_error();
  if (!bytes) return fail(SFT_EINVAL, "sft_ft_fwd_i16_packed_workspace_size: null pointer");
  if (batch < 0 || max_active < 0 || max_active >= 65536 || (perspectives != 1 && perspectives != 2))
    return fail(SFT_EINVAL, "sft_ft_fwd_i16_packed_workspace_size: need batch >= 0, 0 <= max_active < 65536 and "
                            "perspectives 1 or 2");
  *bytes = fwd_i16_ranked_workspace(batch, max_active, perspectives);
  return SFT_OK;
}

int sft_ft_fwd_i16_packed_ex(const int32_t *idx0, const int32_t *idx1, int64_t batch, int32_t max_active,
                             const void *packed, size_t packed_bytes, int64_t num_inputs, int32_t output_size,
                             const int16_t *bias, int32_t psqt_size, int16_t *out0, int16_t *out1, int32_t *psqt_out0,
                             int32_t *psqt_out1, int32_t clip_lo, int32_t clip_hi, void *workspace,
                             size_t workspace_bytes, uint32_t flags, void *stream) {
  clear_error();
  const char *w = "sft_ft_fwd_i16_packed_ex";
  const int rc = check_i16_packed_call(w, idx0, idx1, batch, max_active, packed, packed_bytes, num_inputs, output_size,
                                       bias, psqt_size, out0, out1, psqt_out0, psqt_out1, clip_lo, clip_hi, flags);
  if (rc != SFT_OK) return rc;
  return fwd_i16_packed_ranked(idx0, idx1, batch, max_active, packed, num_inputs, output_size, bias, psqt_size, out0,
                               out1, psqt_size > 0 ? psqt_out0 : nullptr, psqt_size > 0 ? psqt_out1 : nullptr,
                               clip_lo, clip_hi, (flags & SFT_Q16_WRAP16) ? 1 : 0, workspace, workspace_bytes,
                               (hipStream_t)stream, w);
}

int sft_quantize_i16(const float *x, int64_t n, float scale, int16_t *out, void *stream) {
  clear_error();
  if (n < 0) return fail(SFT_EINVAL, "sft_quantize_i16: n must be >= 0");
  if (n > 0 && (!x || !out)) return fail(SFT_EINVAL, "sft_quantize_i16: null pointer");
  return quantize_i16(x, n, scale, out, (hipStream_t)stream);
}

int sft_prof_enable(int on) {
  clear_error();
  std::lock_guard<std::mutex> lock(g_prof_mu);
  drop_pending_locked();
  g_prof_on.store(on != 0);
  return SFT_OK;
}

int sft_prof_num_kinds(void) { return kProfNumKinds; }

const char *sft_prof_kind_name(int kind) {
  if (kind < 0 || kind >= kProfNumKinds) return "";
  return kKindNames[kind];
}

int sft_prof_collect(double *total_ms, int64_t *launches, int n_kinds) {
  clear_error();
  if (!total_ms || !launches || n_kinds < 0) return fail(SFT_EINVAL, "sft_prof_collect: bad arguments");
  std::lock_guard<std::mutex> lock(g_prof_mu);
  int rc = SFT_OK;
  for (auto &p : g_pending) {
    if (hipEventSynchronize(p.stop) != hipSuccess) {
      rc = fail(SFT_EHIP, "sft_prof_collect: event wait failed");
      continue;
    }
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, p.start, p.stop) != hipSuccess) {
      rc = fail(SFT_EHIP, "sft_prof_collect: elapsed time failed");
      continue;
    }
    if (p.kind < n_kinds) {
      total_ms[p.kind] += ms;
      launches[p.kind] += 1;
    }
  }
  drop_pending_locked();
  return rc;
}

int sft_probe_l2_gather(const float *table, int64_t table_rows, int32_t rounds, int32_t blocks, float *out,
                        size_t out_bytes, void *stream) {
  clear_error();
  const char *w = "sft_probe_l2_gather";
  if (!table || !out) return fail(SFT_EINVAL, std::string(w) + ": null pointer");
  if (table_rows < 1 || table_rows > (1 << 24) || (table_rows & (table_rows - 1)) != 0)
    return fail(SFT_EINVAL, std::string(w) + ": table_rows must be a power of two in [1, 2^24]");
  if (rounds < 1 || blocks < 1 || blocks > (1 << 20))
    return fail(SFT_EINVAL, std::string(w) + ": need rounds >= 1 and 1 <= blocks <= 2^20");
  if (out_bytes < (size_t)blocks * kBlock * 16)
    return fail(SFT_EINVAL, std::string(w) + ": out smaller than blocks * 256 * 16 bytes");
  if ((uintptr_t)table % 16 != 0 || (uintptr_t)out % 16 != 0)
    return fail(SFT_EINVAL, std::string(w) + ": table and out must be 16-byte aligned");
  return probe_l2_gather(table, table_rows, rounds, blocks, out, (hipStream_t)stream);
}

}  // extern "C"
