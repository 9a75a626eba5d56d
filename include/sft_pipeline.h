/*
 * sft_pipeline.h -- C ABI of the host data pipeline (libsft_pipeline.so), the
 * loader side of the FT's input contract.
 *
 * Replaces the part of the reference's Rust loader that precedes feature
 * encoding (rgodha24/stockfish-trainer, src/rust/pipeline.rs): the chunk scan
 * with its ".chunks" sidecar cache (:1011-1120), the rank sharding of the chunk
 * list (scan_chunk_tasks, :991-1010), the seeded shuffle of the chunk order
 * (:265-270), the skip filter (SkipDecider, :610-700, 1220-1311), the per-thread
 * shuffle buffer (:707-783) and the pool of host batch slabs (:102-118,
 * 449-592, BatchPipeline::next_batch :351-378).  Feature encoding is not done
 * here: a batch carries the positions (64 piece ids + side to move, 65 bytes
 * each) and sft_encode_features (sft_ft.h) turns them into the FT's index rows
 * on the GPU, where the reference encodes on CPU threads and ships 2 x 4 K
 * bytes of indices per position.
 *
 * Input files hold decoded training entries in chunks:
 *   chunk  = "SFTP" | payload_bytes (u32 LE) | payload_bytes / 72 entries
 *   entry  = sft_entry below (72 bytes, little-endian)
 * (the binpack codec, the sfbinpack crate 0.6.2 the reference links, is not
 * part of this library).
 *
 * Random streams follow the algorithms of the reference's rand 0.8.5 SmallRng
 * (xoshiro256++ seeded by SplitMix64; gen_bool, gen_range and f32 sampling as
 * that crate defines them), so one reader thread with the same seed and the
 * same entry stream makes the same skip and shuffle decisions.
 *
 * Return values: 0 = OK, negative = error (message from
 * sft_pipeline_last_error(), thread-local).  A pipeline object is used from
 * one consumer thread; its worker threads are internal.
 */
#ifndef SFT_PIPELINE_H
#define SFT_PIPELINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SFT_PIPE_OK 0
#define SFT_PIPE_EINVAL (-1)
#define SFT_PIPE_EIO (-2)
#define SFT_PIPE_ECLOSED (-3)

#define SFT_ENTRY_BYTES 72
#define SFT_SQUARE_NONE 64
#define SFT_VALUE_NONE 32002 /* score of an entry without an evaluation */

/* One training entry: the position (piece id per square a1 = 0 .. h8 = 63,
   id = 2 * type + color, pawn..king = 0..5, white = 0, 255 empty), side to
   move (0 white), the move played from it (SFT_SQUARE_NONE when absent), the
   game result from the side to move's view (-1, 0, 1), the score and the ply. */
typedef struct {
  uint8_t board[64];
  uint8_t side_to_move;
  uint8_t move_from;
  uint8_t move_to;
  int8_t result;
  int16_t score;
  uint16_t ply;
} sft_entry;

/* The reference's SkipConfig (src/rust/pipeline.rs:56-67, defaults :227-241). */
typedef struct {
  int32_t filtered;             /* skip captures and positions in check          */
  uint32_t random_fen_skipping; /* skip with probability n / (n + 1)             */
  int32_t wld_filtered;         /* keep with the win/draw/loss model's probability */
  int32_t early_fen_skipping;   /* skip ply <= this (-1: off)                    */
  int32_t simple_eval_skipping; /* skip |material eval| < this (0: off)          */
  int32_t param_index;
  double pc_y1, pc_y2, pc_y3;   /* desired piece-count distribution at 0, 16, 32 */
} sft_skip_config;

typedef struct {
  const char *const *files;
  int32_t num_files;
  int64_t batch_size;
  int32_t reader_threads;         /* chunk readers (skip filter + shuffle buffer each) */
  int32_t slab_count;             /* batch slabs in the pool                         */
  int64_t shuffle_buffer_entries; /* per reader; 0 = no shuffle                      */
  int64_t accumulation_entries;   /* entries a reader hands over at a time           */
  int32_t cyclic;                 /* restart the chunk list forever                  */
  int32_t has_seed;
  uint64_t seed;                  /* chunk order and reader streams (seed ^ reader)  */
  int32_t rank, world_size;       /* keep chunk i when i % world_size == rank        */
  sft_skip_config skip;
} sft_pipeline_config;

/* One batch in a pooled slab: views valid until sft_pipeline_release(slab). */
typedef struct {
  int64_t size;          /* positions in this batch (<= batch_size)            */
  uint8_t *boards;       /* [batch_size][64]                                   */
  uint8_t *side_to_move; /* [batch_size]                                       */
  float *is_white;       /* [batch_size]  1.0 white to move (RowMetadata)      */
  float *outcome;        /* [batch_size]  (result + 1) / 2                     */
  float *score;          /* [batch_size]                                       */
  int32_t slab;          /* pass back to sft_pipeline_release                  */
} sft_batch;

typedef struct {
  uint64_t decoded_entries, skipped_entries, batched_entries, produced_batches, scanned_chunks;
} sft_pipeline_stats;

typedef struct sft_pipeline sft_pipeline;

/* Bytes of one slab for this batch size (the caller may provide the slabs,
   e.g. in pinned host memory for asynchronous copies to the GPU). */
size_t sft_pipeline_slab_bytes(int64_t batch_size);

/* Starts the pipeline.  slab_memory: NULL (the library allocates the slabs) or
   cfg->slab_count pointers to slab_bytes >= sft_pipeline_slab_bytes() each
   (64-byte aligned), owned by the caller until sft_pipeline_destroy. */
int sft_pipeline_create(const sft_pipeline_config *cfg, void *const *slab_memory, size_t slab_bytes,
                        sft_pipeline **out);

/* Next full batch (the last one may be partial): 1 = a batch in *out, 0 = the
   stream has ended, negative = error (a reader failed).  Blocks until one of
   these holds. */
int sft_pipeline_next(sft_pipeline *p, sft_batch *out);

/* Returns a slab to the pool (its batch views become invalid). */
int sft_pipeline_release(sft_pipeline *p, int32_t slab);

int sft_pipeline_stats_get(sft_pipeline *p, sft_pipeline_stats *out);

/* Stops the workers and frees the pipeline (and the slabs it allocated). */
void sft_pipeline_destroy(sft_pipeline *p);

const char *sft_pipeline_last_error(void);

/* Writes n entries to path as chunks of at most entries_per_chunk entries. */
int sft_entries_write(const char *path, const sft_entry *entries, int64_t n, int64_t entries_per_chunk);

/* Chunk list of a file (as the pipeline scans it, through the sidecar cache
   "<path>.chunks" when valid, writing it otherwise): *count chunks, payload
   offsets and entry counts into offsets / counts when not NULL (capacity
   entries at most). */
int sft_chunks_scan(const char *path, int64_t *offsets, int64_t *counts, int64_t capacity, int64_t *count);

/* The skip filter alone over n entries, in order, with one random stream
   seeded by seed: skip[i] = 1 when entry i is skipped. */
int sft_skip_filter(const sft_skip_config *cfg, const sft_entry *entries, int64_t n, uint64_t seed,
                    uint8_t *skip);

/* The random stream: n values of the generator seeded by seed (SplitMix64
   seeding) or, when state is not NULL, started from that 4-word state. */
int sft_rng_u64(uint64_t seed, const uint64_t *state, uint64_t *out, int64_t n);

#ifdef __cplusplus
}
#endif

#endif /* SFT_PIPELINE_H */
