/*
 * slha_eventlog.h — the CCOS EventLog (COLD eviction and rehydrate) over the
 * device arena.
 *
 * Wire format (scirust/src/eventlog.rs:9-36, little-endian):
 *   header 16 B: u32 magic 0x534C4C47 ("SLLG"), u32 version (1 or 2),
 *                u32 tile_size = 128, u32 reserved = 0;
 *   record 144 B: u64 seq, u32 slot, u32 checksum, 128 tile bytes.
 * Version 2's checksum is FNV-1a 32 over seq || slot || tile
 * (eventlog.rs:148-170); version 1 stores 0 there. The tile bytes of a record
 * are the tile's own 128 bytes (`tile_to_bytes`, eventlog.rs:82-100, writes
 * the fields in the struct's byte map), so eviction is a gather on the GPU and
 * rehydrate a checked scatter. The host part keeps the reference's file
 * semantics: no timestamps (identical appends give identical files), strict
 * open, open with recovery of a torn tail record, read-only open, append with
 * optional fsync, lookups of the latest record by seq or slot.
 */
#ifndef SLHA_EVENTLOG_H
#define SLHA_EVENTLOG_H

#include <stddef.h>
#include <stdint.h>

#include "slha.h"

#ifdef __cplusplus
extern "C" {
#endif

#define SLHA_EVENTLOG_MAGIC 0x534C4C47u
#define SLHA_EVENTLOG_VERSION 2u
#define SLHA_EVENTLOG_HEADER_BYTES 16u
#define SLHA_EVENTLOG_RECORD_BYTES 144u

/* slha_eventlog_open modes: EventLog::open (eventlog.rs:240-242),
 * open_recover (:248-250), open_read_only (:256-258). */
#define SLHA_EVENTLOG_OPEN_STRICT 0
#define SLHA_EVENTLOG_OPEN_RECOVER 1
#define SLHA_EVENTLOG_OPEN_READ_ONLY 2

typedef struct SlhaEventLog SlhaEventLog;

/* EventLog::create / create_new (eventlog.rs:193-233): a new version-2 log
 * holding only its header. exclusive != 0 fails if `path` exists; otherwise
 * an existing file is truncated. NULL on failure (last error set). */
SlhaEventLog* slha_eventlog_create(const char* path, int32_t exclusive);

/* EventLog::open_impl (eventlog.rs:260-323): validates the header ("bad
 * magic", "unsupported version", "tile-size mismatch", "file shorter than
 * header"), the record framing ("truncated record"; RECOVER mode instead cuts
 * the partial tail and syncs) and every version-2 checksum ("record checksum
 * mismatch"). NULL on failure. */
SlhaEventLog* slha_eventlog_open(const char* path, int32_t mode);

/* EventLog::append / append_durable (eventlog.rs:330-389) for n records in
 * wire format, as slha_gpu_eventlog_pack writes them with this log's version.
 * Every checksum is checked first (version 2: the FNV-1a; version 1: zero);
 * a bad one appends nothing (SLHA_ERR_INVALID_TILE). A failed write or, with
 * durable != 0, a failed fsync restores the previous length (SLHA_ERR_IO).
 * A read-only log gives SLHA_ERR_IO "EventLog: log opened read-only". */
int32_t slha_eventlog_append(SlhaEventLog* log, const uint8_t* records, size_t n, int32_t durable);

/* EventLog::sync (eventlog.rs:407-410). */
int32_t slha_eventlog_sync(SlhaEventLog* log);

/* EventLog::len (eventlog.rs:392-394) and the log's version; 0 on a bad
 * handle (last error set). */
uint64_t slha_eventlog_len(const SlhaEventLog* log);
uint32_t slha_eventlog_version(const SlhaEventLog* log);

/* EventLog::read_all (eventlog.rs:456-470) over records [first, first + n),
 * in append order, with version-2 checksums checked. */
int32_t slha_eventlog_read(SlhaEventLog* log, uint64_t first, size_t n, uint8_t* records_out);

/* fetch_by_seq / fetch_last_for_slot (eventlog.rs:475-486): the index of the
 * most recently appended record with that seq (slot); *found = 0 when there
 * is none. Like the reference, the scan checks every record. */
int32_t slha_eventlog_find_seq(SlhaEventLog* log, uint64_t seq, uint64_t* index_out, int32_t* found);
int32_t slha_eventlog_find_slot(SlhaEventLog* log, uint32_t slot, uint64_t* index_out, int32_t* found);

/* Closes the file and releases the handle. Calls on one handle are
 * serialised by the library, but none may still be starting on it when it is
 * closed, nor start after. */
int32_t slha_eventlog_close(SlhaEventLog* log);

/* Device side. ElasticKvCache::evict (ccos.rs:404-438) appends
 * (seq[slot], slot, tiles[slot]) per evicted slot: this packs n such records
 * from the arena into records_dev (n * 144 B, 16-byte aligned), with the
 * checksum of `version` (1 or 2). slots_dev / seqs_dev: u32 / u64 [n]. */
int32_t slha_gpu_eventlog_pack(const SciRustSlhaTile* arena_dev, const uint32_t* slots_dev,
                               const uint64_t* seqs_dev, size_t n, uint32_t version,
                               uint8_t* records_dev, void* stream);

/* ElasticKvCache::rehydrate (ccos.rs:451-466) places a logged tile in a free
 * slot: record i's tile goes to arena slot dst_slots_dev[i] when its
 * version-2 checksum holds (status 0); otherwise the slot is not written and
 * status_dev[i] = 1. Version 1 records are not checked. The caller picks the
 * slots (its free list) and the tile's WARM flag gives its state. */
int32_t slha_gpu_eventlog_unpack(const uint8_t* records_dev, size_t n, uint32_t version,
                                 const uint32_t* dst_slots_dev, SciRustSlhaTile* arena_dev,
                                 uint32_t* status_dev, void* stream);

#ifdef __cplusplus
}
#endif
#endif
