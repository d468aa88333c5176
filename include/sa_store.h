/* sa_store.h — the main KV store on local disk, host side (no HIP types).
 *
 * Layout of the reference's main store: one file, a reserved segment of
 * blocks_per_layer blocks per layer, block `block` of layer `layer` at byte
 * (layer * blocks_per_layer + block) * block_bytes
 * (cpp/src/kv_lifecycle_main.cpp:73-80 and :105-108 with blocks_per_layer =
 * capacity_blocks and block = initial_blocks + sealed index;
 * cpp/src/pipeline_main.cpp:660-678 for the reads).  Writes and reads go
 * through O_DIRECT when the file system allows it (block_bytes then needs
 * to be a multiple of 4096; a buffer O_DIRECT cannot use, unaligned or
 * mapped by the GPU driver as hipHostMalloc memory is, goes through a
 * page-aligned bounce buffer of the I/O thread), issued by a small pool of worker threads so that several blocks are in
 * flight at once (the reference queues them on io_uring,
 * cpp/src/uring_reader.cpp:78-122).
 *
 * Errors: a negative return code; the message is sa_hip_last_error()
 * (include/sa_hip.h). */
#ifndef SA_STORE_H_
#define SA_STORE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct sa_store sa_store;

enum {
  SA_STORE_CREATE = 1, /* create or truncate, then reserve layers * blocks_per_layer blocks */
  SA_STORE_DIRECT = 2  /* O_DIRECT when the file system supports it */
};

/* Opens (or creates) the store; `threads` I/O workers (1..64).  NULL on
 * error. */
sa_store* sa_store_open(const char* path, int64_t layers, int64_t blocks_per_layer, int64_t block_bytes,
                        int32_t flags, int32_t threads);
void sa_store_close(sa_store* store);
/* 1 when the file is open with O_DIRECT. */
int sa_store_is_direct(const sa_store* store);
int64_t sa_store_bytes(const sa_store* store);
/* Block transfers that went through a bounce buffer: O_DIRECT cannot use
 * memory the GPU driver mapped (hipHostMalloc), so such blocks are copied
 * through a page-aligned buffer of the I/O thread. */
int64_t sa_store_bounced(const sa_store* store);

/* Queue the reads of blocks[0..count) of `layer` into dst + i * block_bytes
 * (or the writes from src + i * block_bytes); returns a batch id > 0 at
 * once.  Block ids outside [0, blocks_per_layer) or a layer outside
 * [0, layers) are refused before anything is queued. */
int64_t sa_store_submit_reads(sa_store* store, int64_t layer, const int64_t* blocks, int32_t count, void* dst);
int64_t sa_store_submit_writes(sa_store* store, int64_t layer, const int64_t* blocks, int32_t count,
                               const void* src);
/* Wait for a batch; 0, or the first I/O error of the batch. */
int sa_store_wait(sa_store* store, int64_t batch);
/* submit + wait. */
int sa_store_read_blocks(sa_store* store, int64_t layer, const int64_t* blocks, int32_t count, void* dst);
int sa_store_write_blocks(sa_store* store, int64_t layer, const int64_t* blocks, int32_t count, const void* src);
/* fsync of the store file. */
int sa_store_sync(sa_store* store);

/* Crash-consistent commit marker (cpp/src/online_seal_main.cpp:59-70):
 * body is written to directory/name.tmp, fsynced, renamed onto
 * directory/name, and the directory is fsynced, so a reader sees the old
 * marker or the whole new one. */
int sa_store_commit_marker(const char* directory, const char* name, const char* body);

#ifdef __cplusplus
}
#endif

#endif /* SA_STORE_H_ */
