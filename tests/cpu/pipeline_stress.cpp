// Drives the host data pipeline (csrc/host/pipeline.cpp, include/sft_pipeline.h)
// through the paths its threads take: finite, skip-filtered and cyclic streams,
// 4-6 reader threads, caller-provided slabs, destruction right after creation,
// mid-stream and with slabs still held, and a reader that fails mid-stream (its
// file truncated under it) reported to the consumer as the reference's
// take_error_if_any does (src/rust/pipeline.rs:395-410).  Built together with
// the pipeline source under -fsanitize=thread and under
// -fsanitize=address,undefined; any sanitizer report fails the run.  Prints
// "all checks passed" at the end.

#include <unistd.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "sft_pipeline.h"

namespace {

int g_failures = 0;

void check(bool ok, const char *what, int line) {
  if (!ok) {
    std::printf("FAILED line %d: %s (%s)\n", line, what, sft_pipeline_last_error());
    ++g_failures;
  }
}
#define CHECK(cond) check((cond), #cond, __LINE__)

std::vector<sft_entry> make_entries(int64_t n, uint64_t seed) {
  std::mt19937_64 g(seed);
  std::vector<sft_entry> v((size_t)n);
  for (int64_t i = 0; i < n; ++i) {
    sft_entry &e = v[(size_t)i];
    std::memset(e.board, 255, 64);
    const int wk = (int)(g() % 64);
    int bk = (int)(g() % 64);
    if (bk == wk) bk = (wk + 9) % 64;
    e.board[wk] = 10;  // white king
    e.board[bk] = 11;  // black king
    const int extra = (int)(g() % 20);
    for (int k = 0; k < extra; ++k) {
      const int sq = (int)(g() % 64);
      if (e.board[sq] == 255) e.board[sq] = (uint8_t)(g() % 10);  // pawn .. queen, either colour
    }
    e.side_to_move = (uint8_t)(g() & 1);
    e.move_from = SFT_SQUARE_NONE;
    e.move_to = SFT_SQUARE_NONE;
    e.result = (int8_t)((int)(g() % 3) - 1);
    e.score = (int16_t)((int)(g() % 2001) - 1000);
    e.ply = (uint16_t)(g() % 200);
  }
  return v;
}

sft_pipeline_config base_config(const char *const *files, int nfiles, int readers) {
  sft_pipeline_config c;
  std::memset(&c, 0, sizeof(c));
  c.files = files;
  c.num_files = nfiles;
  c.batch_size = 256;
  c.reader_threads = readers;
  c.slab_count = 4;
  c.shuffle_buffer_entries = 1000;
  c.accumulation_entries = 128;
  c.cyclic = 0;
  c.has_seed = 1;
  c.seed = 1234;
  c.rank = 0;
  c.world_size = 1;
  c.skip.early_fen_skipping = -1;
  c.skip.pc_y1 = c.skip.pc_y2 = c.skip.pc_y3 = 1.0;
  return c;
}

// Every entry once: count and score sum over all batches, and the stats.
void finite_stream(const char *path, const std::vector<sft_entry> &entries, int readers, bool own_slabs) {
  const char *files[] = {path};
  sft_pipeline_config c = base_config(files, 1, readers);
  std::vector<void *> slabs;
  const size_t sb = sft_pipeline_slab_bytes(c.batch_size);
  if (own_slabs)
    for (int i = 0; i < c.slab_count; ++i) slabs.push_back(std::aligned_alloc(64, (sb + 63) / 64 * 64));
  sft_pipeline *p = nullptr;
  CHECK(sft_pipeline_create(&c, own_slabs ? slabs.data() : nullptr, sb, &p) == SFT_PIPE_OK);
  if (!p) return;
  int64_t count = 0;
  double score = 0.0;
  sft_batch b;
  int rc;
  while ((rc = sft_pipeline_next(p, &b)) == 1) {
    CHECK(b.size > 0 && b.size <= c.batch_size);
    for (int64_t i = 0; i < b.size; ++i) score += b.score[i];
    count += b.size;
    CHECK(sft_pipeline_release(p, b.slab) == SFT_PIPE_OK);
  }
  CHECK(rc == 0);
  double want = 0.0;
  for (const sft_entry &e : entries) want += e.score;
  CHECK(count == (int64_t)entries.size());
  CHECK(score == want);
  sft_pipeline_stats st;
  CHECK(sft_pipeline_stats_get(p, &st) == SFT_PIPE_OK);
  CHECK(st.decoded_entries == entries.size() && st.skipped_entries == 0 && st.batched_entries == entries.size());
  sft_pipeline_destroy(p);
  for (void *s : slabs) std::free(s);
}

// Skip filter on: batched + skipped == decoded == every entry.
void skip_filtered_stream(const char *path, int64_t n, int readers) {
  const char *files[] = {path};
  sft_pipeline_config c = base_config(files, 1, readers);
  c.skip.random_fen_skipping = 2;
  c.skip.early_fen_skipping = 20;
  c.skip.simple_eval_skipping = 3;
  c.skip.pc_y1 = 1.0;
  c.skip.pc_y2 = 2.0;
  c.skip.pc_y3 = 1.0;
  sft_pipeline *p = nullptr;
  CHECK(sft_pipeline_create(&c, nullptr, 0, &p) == SFT_PIPE_OK);
  if (!p) return;
  int64_t count = 0;
  sft_batch b;
  int rc;
  while ((rc = sft_pipeline_next(p, &b)) == 1) {
    count += b.size;
    CHECK(sft_pipeline_release(p, b.slab) == SFT_PIPE_OK);
  }
  CHECK(rc == 0);
  sft_pipeline_stats st;
  CHECK(sft_pipeline_stats_get(p, &st) == SFT_PIPE_OK);
  CHECK((int64_t)st.decoded_entries == n);
  CHECK(st.skipped_entries > 0 && st.batched_entries + st.skipped_entries == st.decoded_entries);
  CHECK(count == (int64_t)st.batched_entries);
  sft_pipeline_destroy(p);
}

// Cyclic: take batches, keep some slabs, destroy while the readers run.
void cyclic_destroyed_mid_stream(const char *path, int readers, int batches, int held) {
  const char *files[] = {path};
  sft_pipeline_config c = base_config(files, 1, readers);
  c.cyclic = 1;
  c.slab_count = held + 2;
  sft_pipeline *p = nullptr;
  CHECK(sft_pipeline_create(&c, nullptr, 0, &p) == SFT_PIPE_OK);
  if (!p) return;
  sft_batch b;
  for (int i = 0; i < batches; ++i) {
    CHECK(sft_pipeline_next(p, &b) == 1);
    CHECK(b.size == c.batch_size);  // a cyclic stream has no partial batch
    if (i < batches - held) CHECK(sft_pipeline_release(p, b.slab) == SFT_PIPE_OK);
  }
  sft_pipeline_destroy(p);  // `held` slabs never released, readers blocked on a full queue
}

// Destroyed before the consumer asks for anything (readers just started).
void destroyed_at_once(const char *path, int readers) {
  const char *files[] = {path, path};
  sft_pipeline_config c = base_config(files, 2, readers);
  for (int i = 0; i < 20; ++i) {
    sft_pipeline *p = nullptr;
    c.seed = (uint64_t)i;
    c.cyclic = i & 1;
    CHECK(sft_pipeline_create(&c, nullptr, 0, &p) == SFT_PIPE_OK);
    if (i % 3 == 0 && p) {
      sft_batch b;
      CHECK(sft_pipeline_next(p, &b) == 1);
    }
    sft_pipeline_destroy(p);
  }
}

// A reader fails mid-stream: the file loses most of its chunks after the scan,
// while the readers are held back by the bounded queues; the consumer gets
// SFT_PIPE_EIO with the reader's message, and the pipeline is destroyed.
void reader_error_mid_stream(const char *path, const std::vector<sft_entry> &entries, int readers) {
  if (sft_entries_write(path, entries.data(), (int64_t)entries.size(), 500) != SFT_PIPE_OK) {
    CHECK(false);
    return;
  }
  const char *files[] = {path};
  sft_pipeline_config c = base_config(files, 1, readers);
  c.batch_size = 32;
  c.slab_count = 2;
  c.accumulation_entries = 16;
  c.shuffle_buffer_entries = 0;
  sft_pipeline *p = nullptr;
  CHECK(sft_pipeline_create(&c, nullptr, 0, &p) == SFT_PIPE_OK);
  if (!p) return;
  // the readers can run ahead by at most the queue (4 (readers + 1) runs of 16),
  // the slabs and one 500-entry chunk each: far less than the 40 000 entries
  CHECK(truncate(path, (off_t)(4 * (8 + 500 * SFT_ENTRY_BYTES))) == 0);
  sft_batch b;
  int rc;
  int64_t got = 0;
  while ((rc = sft_pipeline_next(p, &b)) == 1) {
    got += b.size;
    CHECK(sft_pipeline_release(p, b.slab) == SFT_PIPE_OK);
  }
  CHECK(rc == SFT_PIPE_EIO);
  CHECK(std::strstr(sft_pipeline_last_error(), "failed to read chunk") != nullptr);
  CHECK(got < (int64_t)entries.size());
  CHECK(sft_pipeline_next(p, &b) == SFT_PIPE_EIO);  // the error stays
  sft_pipeline_destroy(p);
}

}  // namespace

int main(int argc, char **argv) {
  const std::string dir = argc > 1 ? argv[1] : "/tmp";
  const std::string path = dir + "/stress.sftpos", bad = dir + "/truncated.sftpos";
  const std::vector<sft_entry> entries = make_entries(20000, 7);
  if (sft_entries_write(path.c_str(), entries.data(), (int64_t)entries.size(), 500) != SFT_PIPE_OK) {
    std::printf("cannot write %s: %s\n", path.c_str(), sft_pipeline_last_error());
    return 1;
  }
  for (int readers : {4, 6}) {
    finite_stream(path.c_str(), entries, readers, false);
    finite_stream(path.c_str(), entries, readers, true);
    skip_filtered_stream(path.c_str(), (int64_t)entries.size(), readers);
    cyclic_destroyed_mid_stream(path.c_str(), readers, 200, 2);
    destroyed_at_once(path.c_str(), readers);
  }
  reader_error_mid_stream(bad.c_str(), make_entries(40000, 8), 5);
  if (g_failures) {
    std::printf("%d checks failed\n", g_failures);
    return 1;
  }
  std::printf("all checks passed\n");
  return 0;
}
