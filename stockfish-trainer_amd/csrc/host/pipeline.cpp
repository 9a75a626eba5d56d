// Host data pipeline (libsft_pipeline.so, include/sft_pipeline.h): chunk scan
// with a sidecar cache, rank sharding and a seeded chunk order, reader threads
// that apply the skip filter and a shuffle buffer, and an assembler thread that
// fills pooled batch slabs with positions for the GPU encoder.
//
// Stages (the reference's decode stage, src/rust/pipeline.rs:707-783, without
// the binpack codec; its encode stage, :811-863, becomes the slab assembly):
//   readers (reader_threads): claim chunk tasks in the shuffled order (cyclic
//     or once), read the chunk's entries, run SkipDecider, pass the survivors
//     through the shuffle buffer and hand them over in runs of
//     accumulation_entries to the decoded queue;
//   assembler: copies entries into the slab taken from the free queue, moves
//     full slabs (and the last partial one) to the ready queue;
//   consumer: sft_pipeline_next pops the ready queue, sft_pipeline_release
//     returns the slab to the free queue.
// The queues are bounded and closable; closing the decoded queue after the
// last reader and the ready queue after the assembler ends the stream.
#include "sft_pipeline.h"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <memory>
#include <mutex>
#include <random>
#include <string>
#include <thread>
#include <vector>

namespace {

thread_local std::string t_error;
int fail(int code, const std::string &msg) {
  t_error = msg;
  return code;
}

static_assert(sizeof(sft_entry) == SFT_ENTRY_BYTES, "entry records are 72 bytes");

constexpr uint8_t kEmpty = 255;
constexpr uint32_t kMaxChunkBytes = 100u * 1024 * 1024;  // as the reference's BINPACK_MAX_CHUNK_SIZE
constexpr double kMaxSkipRate = 10.0;
constexpr int kWldMaxPly = 240;
constexpr float kWldScoreScale = 100.0f / 208.0f;

// ------------------------------------------------------------ random stream ----
// rand 0.8.5's SmallRng on 64-bit targets: xoshiro256++ (Blackman & Vigna),
// seeded from a u64 by SplitMix64; Bernoulli, uniform-integer and f32 sampling
// as rand 0.8 implements them.
inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
struct SmallRng {
  uint64_t s[4];
  static SmallRng from_u64(uint64_t state) {
    SmallRng r{};
    for (uint64_t &w : r.s) {
      state += 0x9e3779b97f4a7c15ull;
      uint64_t z = state;
      z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
      z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
      w = z ^ (z >> 31);
    }
    if ((r.s[0] | r.s[1] | r.s[2] | r.s[3]) == 0) return from_u64(0);
    return r;
  }
  uint64_t next_u64() {
    const uint64_t result = rotl(s[0] + s[3], 23) + s[0];
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return result;
  }
  uint32_t next_u32() { return (uint32_t)(next_u64() >> 32); }  // the upper bits
  // Bernoulli(p): p == 1 draws nothing; otherwise one u64 below p * 2^64.
  bool gen_bool(double p) {
    if (p == 1.0) return true;
    const uint64_t p_int = (uint64_t)(p * 18446744073709551616.0);
    return next_u64() < p_int;
  }
  float gen_f32() { return (float)(next_u32() >> 8) * (1.0f / 16777216.0f); }
  // Uniform in [0, n) (n >= 1): widening multiply with the conservative zone.
  uint64_t gen_range_u64(uint64_t n) {
    const uint64_t zone = (n << __builtin_clzll(n)) - 1;
    for (;;) {
      const unsigned __int128 m = (unsigned __int128)next_u64() * n;
      if ((uint64_t)m <= zone) return (uint64_t)(m >> 64);
    }
  }
  uint32_t gen_range_u32(uint32_t n) {
    const uint32_t zone = (n << __builtin_clz(n)) - 1;
    for (;;) {
      const uint64_t m = (uint64_t)next_u32() * n;
      if ((uint32_t)m <= zone) return (uint32_t)(m >> 32);
    }
  }
  // rand's slice shuffle: for i = len-1 .. 1, swap(i, uniform [0, i]).
  template <typename T>
  void shuffle(std::vector<T> &v) {
    for (size_t i = v.size(); i-- > 1;) {
      const size_t j = (i + 1) <= 0xffffffffu ? gen_range_u32((uint32_t)(i + 1)) : gen_range_u64(i + 1);
      std::swap(v[i], v[j]);
    }
  }
};

// ------------------------------------------------------------- chess bits ----
int type_of(uint8_t p) { return p / 2; }
int color_of(uint8_t p) { return p % 2; }

// Whether square sq is attacked by a piece of colour `by` on board b.
bool attacked_by(const uint8_t *b, int sq, int by) {
  const int f0 = sq % 8, r0 = sq / 8;
  auto piece = [&](int f, int r) -> int { return (f < 0 || f > 7 || r < 0 || r > 7) ? -1 : b[r * 8 + f]; };
  // pawns of colour `by` attack diagonally forward from their side
  const int pr = by == 0 ? r0 - 1 : r0 + 1;
  for (int df : {-1, 1}) {
    const int p = piece(f0 + df, pr);
    if (p >= 0 && p != kEmpty && type_of(p) == 0 && color_of(p) == by) return true;
  }
  static const int kn[8][2] = {{1, 2}, {2, 1}, {2, -1}, {1, -2}, {-1, -2}, {-2, -1}, {-2, 1}, {-1, 2}};
  for (const auto &d : kn) {
    const int p = piece(f0 + d[0], r0 + d[1]);
    if (p >= 0 && p != kEmpty && type_of(p) == 1 && color_of(p) == by) return true;
  }
  static const int kg[8][2] = {{1, 0}, {1, 1}, {0, 1}, {-1, 1}, {-1, 0}, {-1, -1}, {0, -1}, {1, -1}};
  for (const auto &d : kg) {
    const int p = piece(f0 + d[0], r0 + d[1]);
    if (p >= 0 && p != kEmpty && type_of(p) == 5 && color_of(p) == by) return true;
  }
  for (int k = 0; k < 8; ++k) {  // rays: k < 4 orthogonal (rook, queen), else diagonal (bishop, queen)
    const int df = kg[k][0], dr = kg[k][1];
    const bool diag = df != 0 && dr != 0;
    for (int f = f0 + df, r = r0 + dr; f >= 0 && f < 8 && r >= 0 && r < 8; f += df, r += dr) {
      const int p = b[r * 8 + f];
      if (p == kEmpty) continue;
      if (color_of(p) == by && (type_of(p) == 4 || type_of(p) == (diag ? 2 : 3))) return true;
      break;
    }
  }
  return false;
}

bool is_in_check(const sft_entry &e) {
  const int us = e.side_to_move & 1;
  for (int sq = 0; sq < 64; ++sq)
    if (e.board[sq] == 2 * 5 + us) return attacked_by(e.board, sq, us ^ 1);
  return false;
}

// A capture by the entry's move: a piece of the other colour on its target.
// An empty source square counts as white (sfbinpack's Piece::none() colour).
bool is_capturing_move(const sft_entry &e) {
  if (e.move_from >= 64 || e.move_to >= 64) return false;
  const uint8_t captured = e.board[e.move_to], moving = e.board[e.move_from];
  const int moving_color = moving == kEmpty ? 0 : color_of(moving);
  return captured != kEmpty && color_of(captured) != moving_color;
}

int piece_count(const sft_entry &e) {
  int n = 0;
  for (uint8_t p : e.board) n += p != kEmpty;
  return n;
}

// Material balance from the side to move's view (src/rust/pipeline.rs:1254-1271).
int simple_eval(const sft_entry &e) {
  static const int value[5] = {208, 781, 825, 1276, 2538};
  int v = 0;
  for (uint8_t p : e.board)
    if (p != kEmpty && type_of(p) < 5) v += color_of(p) == 0 ? value[type_of(p)] : -value[type_of(p)];
  return (e.side_to_move & 1) == 0 ? v : -v;
}

// ------------------------------------------------------------ skip filter ----
struct WldParams {
  float a, inv_b;
};
const std::vector<WldParams> &wld_params() {
  static const std::vector<WldParams> params = [] {
    const float as[4] = {-3.683893f, 30.07066f, -60.52879f, 149.53378f};
    const float bs[4] = {-2.0181856f, 15.856851f, -29.83452f, 47.59079f};
    std::vector<WldParams> v;
    for (int ply = 0; ply <= kWldMaxPly; ++ply) {
      const float m = (float)ply / 64.0f;
      const float a = (((as[0] * m + as[1]) * m + as[2]) * m) + as[3];
      const float b = ((((bs[0] * m + bs[1]) * m + bs[2]) * m) + bs[3]) * 1.5f;
      v.push_back(WldParams{a, 1.0f / b});
    }
    return v;
  }();
  return params;
}

// Probability that the game result agrees with the score (pipeline.rs:1281-1294).
float score_result_prob(const sft_entry &e) {
  const WldParams &p = wld_params()[e.ply < kWldMaxPly ? e.ply : kWldMaxPly];
  float x = (float)e.score * kWldScoreScale;
  x = x < -2000.0f ? -2000.0f : (x > 2000.0f ? 2000.0f : x);
  if (e.result > 0) return 1.0f / (1.0f + std::exp((p.a - x) * p.inv_b));
  if (e.result < 0) return 1.0f / (1.0f + std::exp((p.a + x) * p.inv_b));
  const float w = 1.0f / (1.0f + std::exp((p.a - x) * p.inv_b));
  const float l = 1.0f / (1.0f + std::exp((p.a + x) * p.inv_b));
  const float d = 1.0f - w - l;
  return d > 0.0f ? d : 0.0f;
}

// Lagrange interpolation through (0, y1), (16, y2), (32, y3) (pipeline.rs:1220-1233).
double desired_piece_count_weight(const sft_skip_config &c, int n) {
  const double x = n, x1 = 0.0, x2 = 16.0, x3 = 32.0;
  const double l1 = (x - x2) * (x - x3) / ((x1 - x2) * (x1 - x3));
  const double l2 = (x - x1) * (x - x3) / ((x2 - x1) * (x2 - x3));
  const double l3 = (x - x1) * (x - x2) / ((x3 - x1) * (x3 - x2));
  return l1 * c.pc_y1 + l2 * c.pc_y2 + l3 * c.pc_y3;
}

// SkipDecider (pipeline.rs:610-700): the same rules, in the same order, with
// the same draws from the stream.
struct SkipDecider {
  bool enabled;
  sft_skip_config cfg;
  double random_skip_probability, weights_total, alpha = 1.0;
  double hist_all[33] = {}, hist_passed[33] = {};
  double all_total = 0.0, passed_total = 0.0;

  explicit SkipDecider(const sft_skip_config &c) : cfg(c) {
    enabled = c.filtered || c.random_fen_skipping > 0 || c.wld_filtered || c.early_fen_skipping >= 0;
    random_skip_probability =
        c.random_fen_skipping == 0 ? 0.0 : (double)c.random_fen_skipping / ((double)c.random_fen_skipping + 1.0);
    weights_total = 0.0;
    for (int n = 0; n <= 32; ++n) weights_total += desired_piece_count_weight(c, n);
  }

  bool should_skip(const sft_entry &e, SmallRng &rng) {
    if (!enabled) return false;
    if (e.score == SFT_VALUE_NONE) return true;
    if ((int)e.ply <= cfg.early_fen_skipping) return true;
    if (cfg.random_fen_skipping > 0 && rng.gen_bool(random_skip_probability)) return true;
    if (cfg.wld_filtered) {
      const float keep = score_result_prob(e);
      if (keep <= 0.0f || (keep < 1.0f && rng.gen_f32() >= keep)) return true;
    }
    if (cfg.filtered && (is_capturing_move(e) || is_in_check(e))) return true;
    if (cfg.simple_eval_skipping > 0 && std::abs(simple_eval(e)) < cfg.simple_eval_skipping) return true;

    int pc = piece_count(e);
    if (pc > 32) pc = 32;  // no chess position holds more
    hist_all[pc] += 1.0;
    all_total += 1.0;
    if ((uint64_t)all_total % 10000 == 0) {
      double pass = all_total * weights_total;
      for (int i = 0; i <= 32; ++i) {
        const double w = desired_piece_count_weight(cfg, i);
        if (w > 0.0 && hist_all[i] > 0.0) {
          const double tmp = all_total * w / (weights_total * hist_all[i]);
          if (tmp < pass) pass = tmp;
        }
      }
      alpha = 1.0 / (pass * kMaxSkipRate);
    }
    double tmp = alpha * all_total * desired_piece_count_weight(cfg, pc) / (weights_total * hist_all[pc]);
    if (tmp > 1.0) tmp = 1.0;
    double p = 1.0 - tmp;
    p = p < 0.0 ? 0.0 : (p > 1.0 ? 1.0 : p);
    if (rng.gen_bool(p)) return true;
    hist_passed[pc] += 1.0;
    passed_total += 1.0;
    return false;
  }
};

// ------------------------------------------------------------- chunk scan ----
struct ChunkTask {
  int file;
  uint64_t offset;  // of the payload
  uint32_t bytes;
};

constexpr char kChunkMagic[4] = {'S', 'F', 'T', 'P'};
constexpr char kSidecarMagic[4] = {'C', 'H', 'N', 'K'};
constexpr uint32_t kSidecarVersion = 1;
constexpr size_t kSidecarHeader = 4 + 4 + 8 + 4, kSidecarEntry = 8 + 4;

template <typename T>
void put_le(std::vector<uint8_t> &buf, T v) {
  for (size_t i = 0; i < sizeof(T); ++i) buf.push_back((uint8_t)((uint64_t)v >> (8 * i)));
}
template <typename T>
T get_le(const uint8_t *p) {
  uint64_t v = 0;
  for (size_t i = 0; i < sizeof(T); ++i) v |= (uint64_t)p[i] << (8 * i);
  return (T)v;
}

bool read_all(int fd, uint64_t offset, void *dst, size_t n) {
  uint8_t *d = static_cast<uint8_t *>(dst);
  while (n > 0) {
    const ssize_t r = pread(fd, d, n, (off_t)offset);
    if (r <= 0) return false;
    d += r;
    n -= (size_t)r;
    offset += (uint64_t)r;
  }
  return true;
}

// The sidecar cache "<path>.chunks" (the reference's format, pipeline.rs:1011-1018):
// magic | version u32 | source file size u64 | chunk count u32 | [offset u64, bytes u32]*.
bool load_sidecar(const std::string &path, uint64_t file_size, int file, std::vector<ChunkTask> &out) {
  FILE *f = std::fopen((path + ".chunks").c_str(), "rb");
  if (!f) return false;
  std::vector<uint8_t> d;
  uint8_t buf[4096];
  size_t r;
  while ((r = std::fread(buf, 1, sizeof(buf), f)) > 0) d.insert(d.end(), buf, buf + r);
  std::fclose(f);
  if (d.size() < kSidecarHeader || std::memcmp(d.data(), kSidecarMagic, 4) != 0 ||
      get_le<uint32_t>(d.data() + 4) != kSidecarVersion || get_le<uint64_t>(d.data() + 8) != file_size)
    return false;
  const uint32_t n = get_le<uint32_t>(d.data() + 16);
  if (d.size() != kSidecarHeader + (size_t)n * kSidecarEntry) return false;
  std::vector<ChunkTask> tasks;
  for (uint32_t i = 0; i < n; ++i) {
    const uint8_t *e = d.data() + kSidecarHeader + (size_t)i * kSidecarEntry;
    const ChunkTask t{file, get_le<uint64_t>(e), get_le<uint32_t>(e + 8)};
    if (t.bytes % SFT_ENTRY_BYTES != 0 || t.offset + t.bytes > file_size) return false;
    tasks.push_back(t);
  }
  out.insert(out.end(), tasks.begin(), tasks.end());
  return true;
}

void write_sidecar(const std::string &path, uint64_t file_size, const ChunkTask *tasks, size_t n) {
  std::vector<uint8_t> buf(kSidecarMagic, kSidecarMagic + 4);
  put_le<uint32_t>(buf, kSidecarVersion);
  put_le<uint64_t>(buf, file_size);
  put_le<uint32_t>(buf, (uint32_t)n);
  for (size_t i = 0; i < n; ++i) {
    put_le<uint64_t>(buf, tasks[i].offset);
    put_le<uint32_t>(buf, tasks[i].bytes);
  }
  // write then rename, so a concurrent reader never sees a partial cache
  const std::string tmp = path + ".chunks.tmp." + std::to_string((long)getpid());
  FILE *f = std::fopen(tmp.c_str(), "wb");
  if (!f) return;
  const bool ok = std::fwrite(buf.data(), 1, buf.size(), f) == buf.size();
  if (std::fclose(f) != 0 || !ok || std::rename(tmp.c_str(), (path + ".chunks").c_str()) != 0)
    std::remove(tmp.c_str());
}

int scan_file(const std::string &path, int file, std::vector<ChunkTask> &tasks) {
  struct stat st;
  if (stat(path.c_str(), &st) != 0) return fail(SFT_PIPE_EIO, "cannot stat " + path);
  const uint64_t size = (uint64_t)st.st_size;
  if (load_sidecar(path, size, file, tasks)) return SFT_PIPE_OK;
  const int fd = open(path.c_str(), O_RDONLY);
  if (fd < 0) return fail(SFT_PIPE_EIO, "cannot open " + path);
  const size_t first = tasks.size();
  uint64_t off = 0;
  int rc = SFT_PIPE_OK;
  while (off < size) {
    uint8_t h[8];
    if (off + 8 > size || !read_all(fd, off, h, 8) || std::memcmp(h, kChunkMagic, 4) != 0) {
      rc = fail(SFT_PIPE_EIO, path + ": bad chunk header at offset " + std::to_string(off));
      break;
    }
    const uint32_t bytes = get_le<uint32_t>(h + 4);
    if (bytes > kMaxChunkBytes || bytes % SFT_ENTRY_BYTES != 0 || off + 8 + bytes > size) {
      rc = fail(SFT_PIPE_EIO, path + ": bad chunk size at offset " + std::to_string(off));
      break;
    }
    tasks.push_back(ChunkTask{file, off + 8, bytes});
    off += 8 + bytes;
  }
  close(fd);
  if (rc != SFT_PIPE_OK) {
    tasks.resize(first);
    return rc;
  }
  write_sidecar(path, size, tasks.data() + first, tasks.size() - first);
  return SFT_PIPE_OK;
}

// --------------------------------------------------------- bounded queue ----
template <typename T>
class Queue {
 public:
  explicit Queue(size_t cap) : cap_(cap) {}
  // false when the queue was closed (the item is dropped)
  bool push(T v) {
    std::unique_lock<std::mutex> l(mu_);
    not_full_.wait(l, [&] { return closed_ || q_.size() < cap_; });
    if (closed_) return false;
    q_.push_back(std::move(v));
    not_empty_.notify_one();
    return true;
  }
  // false when the queue is closed and drained
  bool pop(T &v) {
    std::unique_lock<std::mutex> l(mu_);
    not_empty_.wait(l, [&] { return closed_ || !q_.empty(); });
    if (q_.empty()) return false;
    v = std::move(q_.front());
    q_.pop_front();
    not_full_.notify_one();
    return true;
  }
  void close() {
    std::lock_guard<std::mutex> l(mu_);
    closed_ = true;
    not_empty_.notify_all();
    not_full_.notify_all();
  }

 private:
  std::mutex mu_;
  std::condition_variable not_empty_, not_full_;
  std::deque<T> q_;
  size_t cap_;
  bool closed_ = false;
};

// Slab layout: boards [B][64] | side_to_move [B] | is_white [B] f32 | outcome [B] f32 | score [B] f32,
// each array 64-byte aligned.
size_t align64(size_t v) { return (v + 63) & ~(size_t)63; }
struct SlabLayout {
  size_t boards, stm, is_white, outcome, score, total;
  explicit SlabLayout(int64_t B) {
    size_t off = 0;
    boards = off;
    off = align64(off + (size_t)B * 64);
    stm = off;
    off = align64(off + (size_t)B);
    is_white = off;
    off = align64(off + (size_t)B * 4);
    outcome = off;
    off = align64(off + (size_t)B * 4);
    score = off;
    off = align64(off + (size_t)B * 4);
    total = off;
  }
};

}  // namespace

struct sft_pipeline {
  sft_pipeline_config cfg{};
  std::vector<std::string> files;
  std::vector<ChunkTask> tasks;
  std::atomic<uint64_t> next_task{0};
  SlabLayout layout{1};
  std::vector<uint8_t *> slabs;
  std::vector<int64_t> fill;  // entries in each slab
  bool own_slabs = false;

  Queue<std::vector<sft_entry>> decoded;
  Queue<int32_t> free_slabs, ready;
  std::atomic<bool> shutdown{false};
  std::atomic<int> readers_left{0};
  std::mutex err_mu;
  std::string error;
  std::atomic<uint64_t> decoded_entries{0}, skipped_entries{0}, batched_entries{0}, produced_batches{0};
  std::vector<std::thread> workers;

  sft_pipeline(size_t decoded_cap, size_t nslabs) : decoded(decoded_cap), free_slabs(nslabs), ready(nslabs) {}

  void report(const std::string &msg) {
    std::lock_guard<std::mutex> l(err_mu);
    if (error.empty()) error = msg;
  }

  bool claim(ChunkTask &t) {
    if (tasks.empty() || shutdown.load()) return false;
    const uint64_t i = next_task.fetch_add(1);
    if (cfg.cyclic) {
      t = tasks[i % tasks.size()];
      return true;
    }
    if (i >= tasks.size()) return false;
    t = tasks[i];
    return true;
  }

  void reader(int index, uint64_t base_seed) {
    SmallRng rng = SmallRng::from_u64(base_seed ^ (uint64_t)index);
    SkipDecider skip(cfg.skip);
    std::vector<sft_entry> shuffle, acc, chunk;
    const size_t shuffle_cap = (size_t)cfg.shuffle_buffer_entries;
    std::vector<int> fds(files.size(), -1);
    auto hand_over = [&]() -> bool {
      if (acc.empty()) return true;
      std::vector<sft_entry> out;
      out.swap(acc);
      acc.reserve((size_t)cfg.accumulation_entries);
      return decoded.push(std::move(out));
    };
    bool ok = true;
    ChunkTask t;
    while (ok && claim(t)) {
      int &fd = fds[t.file];
      if (fd < 0) fd = open(files[t.file].c_str(), O_RDONLY);
      chunk.resize(t.bytes / SFT_ENTRY_BYTES);
      if (fd < 0 || !read_all(fd, t.offset, chunk.data(), t.bytes)) {
        report("failed to read chunk from " + files[t.file] + " at offset " + std::to_string(t.offset));
        ok = false;
        break;
      }
      uint64_t dec = 0, sk = 0;
      for (const sft_entry &e : chunk) {
        ++dec;
        if (skip.should_skip(e, rng)) {
          ++sk;
          continue;
        }
        if (shuffle_cap == 0) {
          acc.push_back(e);
        } else {
          shuffle.push_back(e);
          if (shuffle.size() >= shuffle_cap) {  // swap_remove at a uniform index
            const size_t j = (size_t)rng.gen_range_u64(shuffle.size());
            acc.push_back(shuffle[j]);
            shuffle[j] = shuffle.back();
            shuffle.pop_back();
          }
        }
        if ((int64_t)acc.size() >= cfg.accumulation_entries && !hand_over()) {
          ok = false;
          break;
        }
      }
      decoded_entries += dec;
      skipped_entries += sk;
    }
    while (ok && !shuffle.empty()) {  // drain the shuffle buffer in random order
      const size_t j = (size_t)rng.gen_range_u64(shuffle.size());
      acc.push_back(shuffle[j]);
      shuffle[j] = shuffle.back();
      shuffle.pop_back();
      if ((int64_t)acc.size() >= cfg.accumulation_entries && !hand_over()) ok = false;
    }
    if (ok) hand_over();
    for (int fd : fds)
      if (fd >= 0) close(fd);
    if (--readers_left == 0) decoded.close();
  }

  void assembler() {
    int32_t cur = -1;
    std::vector<sft_entry> run;
    const int64_t B = cfg.batch_size;
    while (decoded.pop(run)) {
      for (const sft_entry &e : run) {
        if (cur < 0) {
          if (!free_slabs.pop(cur)) {
            ready.close();
            return;
          }
          fill[cur] = 0;
        }
        uint8_t *s = slabs[cur];
        const int64_t i = fill[cur]++;
        std::memcpy(s + layout.boards + (size_t)i * 64, e.board, 64);
        const uint8_t stm = e.side_to_move & 1;
        s[layout.stm + (size_t)i] = stm;
        reinterpret_cast<float *>(s + layout.is_white)[i] = stm == 0 ? 1.0f : 0.0f;
        reinterpret_cast<float *>(s + layout.outcome)[i] = ((float)e.result + 1.0f) / 2.0f;
        reinterpret_cast<float *>(s + layout.score)[i] = (float)e.score;
        ++batched_entries;
        if (fill[cur] == B) {
          ++produced_batches;
          if (!ready.push(cur)) return;
          cur = -1;
        }
      }
    }
    if (cur >= 0 && fill[cur] > 0) {
      ++produced_batches;
      ready.push(cur);
    }
    ready.close();
  }

  void stop() {
    shutdown = true;
    decoded.close();
    free_slabs.close();
    ready.close();
    for (std::thread &t : workers)
      if (t.joinable()) t.join();
    workers.clear();
  }

  ~sft_pipeline() {
    stop();
    if (own_slabs)
      for (uint8_t *s : slabs) std::free(s);
  }
};

extern "C" {

const char *sft_pipeline_last_error(void) { return t_error.c_str(); }

size_t sft_pipeline_slab_bytes(int64_t batch_size) { return batch_size > 0 ? SlabLayout(batch_size).total : 0; }

int sft_pipeline_create(const sft_pipeline_config *cfg, void *const *slab_memory, size_t slab_bytes,
                        sft_pipeline **out) {
  t_error.clear();
  if (!cfg || !out) return fail(SFT_PIPE_EINVAL, "sft_pipeline_create: null pointer");
  *out = nullptr;
  if (cfg->num_files <= 0 || !cfg->files) return fail(SFT_PIPE_EINVAL, "pipeline requires at least one input file");
  if (cfg->batch_size <= 0) return fail(SFT_PIPE_EINVAL, "batch_size must be greater than zero");
  if (cfg->reader_threads <= 0) return fail(SFT_PIPE_EINVAL, "reader_threads must be greater than zero");
  if (cfg->slab_count <= 0) return fail(SFT_PIPE_EINVAL, "slab_count must be greater than zero");
  if (cfg->accumulation_entries <= 0) return fail(SFT_PIPE_EINVAL, "accumulation_entries must be greater than zero");
  if (cfg->shuffle_buffer_entries < 0) return fail(SFT_PIPE_EINVAL, "shuffle_buffer_entries must be >= 0");
  if (cfg->world_size <= 0) return fail(SFT_PIPE_EINVAL, "world_size must be greater than zero");
  if (cfg->rank < 0 || cfg->rank >= cfg->world_size) return fail(SFT_PIPE_EINVAL, "rank must be less than world_size");
  const SlabLayout layout(cfg->batch_size);
  if (slab_memory) {
    if (slab_bytes < layout.total) return fail(SFT_PIPE_EINVAL, "slab_bytes smaller than sft_pipeline_slab_bytes()");
    for (int i = 0; i < cfg->slab_count; ++i)
      if (!slab_memory[i] || (uintptr_t)slab_memory[i] % 64 != 0)
        return fail(SFT_PIPE_EINVAL, "slab memory must be non-null and 64-byte aligned");
  }

  const int readers = cfg->reader_threads;
  auto p = std::make_unique<sft_pipeline>((size_t)std::max(16, 4 * (readers + 1)), (size_t)cfg->slab_count);
  p->cfg = *cfg;
  p->layout = layout;
  for (int i = 0; i < cfg->num_files; ++i) {
    if (!cfg->files[i]) return fail(SFT_PIPE_EINVAL, "null file name");
    p->files.emplace_back(cfg->files[i]);
  }
  p->cfg.files = nullptr;  // the names live in p->files

  // chunk list of every file in order, this rank's share (index % world == rank),
  // then the chunk order shuffled with the seed (pipeline.rs:265-270, 991-1010)
  std::vector<ChunkTask> all;
  for (int i = 0; i < (int)p->files.size(); ++i) {
    const int rc = scan_file(p->files[i], i, all);
    if (rc != SFT_PIPE_OK) return rc;
  }
  for (size_t i = 0; i < all.size(); ++i)
    if ((int64_t)(i % (size_t)cfg->world_size) == cfg->rank) p->tasks.push_back(all[i]);
  const uint64_t seed = cfg->has_seed ? cfg->seed : std::random_device{}() ^ ((uint64_t)std::random_device{}() << 32);
  if (!p->tasks.empty()) {
    SmallRng rng = SmallRng::from_u64(seed);
    rng.shuffle(p->tasks);
  }

  p->slabs.resize(cfg->slab_count);
  p->fill.assign(cfg->slab_count, 0);
  p->own_slabs = slab_memory == nullptr;
  for (int i = 0; i < cfg->slab_count; ++i) {
    p->slabs[i] = slab_memory ? static_cast<uint8_t *>(slab_memory[i])
                              : static_cast<uint8_t *>(std::aligned_alloc(64, layout.total));
    if (!p->slabs[i]) return fail(SFT_PIPE_EINVAL, "slab allocation failed");
    p->free_slabs.push(i);
  }

  p->readers_left = readers;
  for (int i = 0; i < readers; ++i) p->workers.emplace_back(&sft_pipeline::reader, p.get(), i, seed);
  p->workers.emplace_back(&sft_pipeline::assembler, p.get());
  *out = p.release();
  return SFT_PIPE_OK;
}

int sft_pipeline_next(sft_pipeline *p, sft_batch *out) {
  t_error.clear();
  if (!p || !out) return fail(SFT_PIPE_EINVAL, "sft_pipeline_next: null pointer");
  int32_t s = -1;
  const bool got = p->ready.pop(s);
  {
    std::lock_guard<std::mutex> l(p->err_mu);
    if (!p->error.empty()) {
      if (got) p->free_slabs.push(s);
      return fail(SFT_PIPE_EIO, p->error);
    }
  }
  if (!got) return 0;
  uint8_t *base = p->slabs[s];
  out->size = p->fill[s];
  out->boards = base + p->layout.boards;
  out->side_to_move = base + p->layout.stm;
  out->is_white = reinterpret_cast<float *>(base + p->layout.is_white);
  out->outcome = reinterpret_cast<float *>(base + p->layout.outcome);
  out->score = reinterpret_cast<float *>(base + p->layout.score);
  out->slab = s;
  return 1;
}

int sft_pipeline_release(sft_pipeline *p, int32_t slab) {
  t_error.clear();
  if (!p || slab < 0 || slab >= (int32_t)p->slabs.size()) return fail(SFT_PIPE_EINVAL, "sft_pipeline_release: bad slab");
  if (!p->free_slabs.push(slab)) return fail(SFT_PIPE_ECLOSED, "pipeline stopped");
  return SFT_PIPE_OK;
}

int sft_pipeline_stats_get(sft_pipeline *p, sft_pipeline_stats *out) {
  if (!p || !out) return fail(SFT_PIPE_EINVAL, "sft_pipeline_stats_get: null pointer");
  out->decoded_entries = p->decoded_entries.load();
  out->skipped_entries = p->skipped_entries.load();
  out->batched_entries = p->batched_entries.load();
  out->produced_batches = p->produced_batches.load();
  out->scanned_chunks = p->tasks.size();
  return SFT_PIPE_OK;
}

void sft_pipeline_destroy(sft_pipeline *p) { delete p; }

int sft_entries_write(const char *path, const sft_entry *entries, int64_t n, int64_t entries_per_chunk) {
  t_error.clear();
  if (!path || (n > 0 && !entries) || n < 0 || entries_per_chunk <= 0 ||
      entries_per_chunk * SFT_ENTRY_BYTES > (int64_t)kMaxChunkBytes)
    return fail(SFT_PIPE_EINVAL, "sft_entries_write: bad arguments");
  FILE *f = std::fopen(path, "wb");
  if (!f) return fail(SFT_PIPE_EIO, std::string("cannot create ") + path);
  bool ok = true;
  for (int64_t i = 0; i < n && ok; i += entries_per_chunk) {
    const int64_t m = std::min(entries_per_chunk, n - i);
    std::vector<uint8_t> h(kChunkMagic, kChunkMagic + 4);
    put_le<uint32_t>(h, (uint32_t)(m * SFT_ENTRY_BYTES));
    ok = std::fwrite(h.data(), 1, 8, f) == 8 &&
         std::fwrite(entries + i, SFT_ENTRY_BYTES, (size_t)m, f) == (size_t)m;
  }
  if (std::fclose(f) != 0 || !ok) return fail(SFT_PIPE_EIO, std::string("write failed: ") + path);
  return SFT_PIPE_OK;
}

int sft_chunks_scan(const char *path, int64_t *offsets, int64_t *counts, int64_t capacity, int64_t *count) {
  t_error.clear();
  if (!path || !count) return fail(SFT_PIPE_EINVAL, "sft_chunks_scan: null pointer");
  std::vector<ChunkTask> tasks;
  const int rc = scan_file(path, 0, tasks);
  if (rc != SFT_PIPE_OK) return rc;
  *count = (int64_t)tasks.size();
  for (int64_t i = 0; i < (int64_t)tasks.size() && i < capacity; ++i) {
    if (offsets) offsets[i] = (int64_t)tasks[i].offset;
    if (counts) counts[i] = tasks[i].bytes / SFT_ENTRY_BYTES;
  }
  return SFT_PIPE_OK;
}

int sft_skip_filter(const sft_skip_config *cfg, const sft_entry *entries, int64_t n, uint64_t seed, uint8_t *skip) {
  t_error.clear();
  if (!cfg || n < 0 || (n > 0 && (!entries || !skip))) return fail(SFT_PIPE_EINVAL, "sft_skip_filter: bad arguments");
  SmallRng rng = SmallRng::from_u64(seed);
  SkipDecider d(*cfg);
  for (int64_t i = 0; i < n; ++i) skip[i] = d.should_skip(entries[i], rng) ? 1 : 0;
  return SFT_PIPE_OK;
}

int sft_rng_u64(uint64_t seed, const uint64_t *state, uint64_t *out, int64_t n) {
  t_error.clear();
  if (n < 0 || (n > 0 && !out)) return fail(SFT_PIPE_EINVAL, "sft_rng_u64: bad arguments");
  SmallRng rng = SmallRng::from_u64(seed);
  if (state) std::memcpy(rng.s, state, sizeof(rng.s));
  for (int64_t i = 0; i < n; ++i) out[i] = rng.next_u64();
  return SFT_PIPE_OK;
}

}  // extern "C"
