/*
 * slha_ccos.h — CCOS ElasticKvCache (scirust/src/ccos.rs) over a device
 * arena of 128-byte tiles.
 *
 * The tiles stay in HBM. The host keeps the control plane: per-slot state
 * (HOT / WARM / COLD), insertion seq, residual sigma, position and flags, the
 * free list, and the running logical footprint (HOT 128, WARM 96, COLD 0,
 * minus a paged-out TQ3 / MIX3 correction plane of 16 / 14 bytes;
 * ccos.rs:470-482). Every decision follows the reference; the byte changes
 * are device launches: page_out and drop_correction (the kernel of
 * slha_gpu_ccos_apply), eviction records (slha_gpu_eventlog_pack), rehydrate
 * (slha_gpu_eventlog_unpack). H2O importance lives on the device and is
 * accumulated there from the scores of the whole arena.
 *
 * Calls are synchronous on `stream` (they return after their device work is
 * done), as the reference's methods are, except slha_ccos_observe_scores,
 * which only enqueues its kernels: it is called once per decode step, and
 * what it changes (the device importance) is read back only by later calls,
 * which order themselves after it on their stream. Use one stream per cache,
 * or order the streams yourself. One cache is not safe for concurrent calls
 * from several threads.
 */
#ifndef SLHA_CCOS_H
#define SLHA_CCOS_H

#include <stddef.h>
#include <stdint.h>

#include "slha.h"
#include "slha_eventlog.h"

#ifdef __cplusplus
extern "C" {
#endif

/* PageOutPolicy (ccos.rs:44-59). */
#define SLHA_CCOS_PAGE_LOWEST_IMPACT_FIRST 0 /* lowest residual_sigma first (default) */
#define SLHA_CCOS_PAGE_OLDEST_FIRST 1

/* EvictionPolicy (ccos.rs:61-83). */
#define SLHA_CCOS_EVICT_CAUSAL 0     /* oldest seq first (default) */
#define SLHA_CCOS_EVICT_IMPORTANCE 1 /* lowest importance first, sinks last */

/* TileState (ccos.rs:36-41). */
#define SLHA_CCOS_HOT 0
#define SLHA_CCOS_WARM 1
#define SLHA_CCOS_COLD 2

typedef struct SlhaCcos SlhaCcos;

typedef struct {
    uint64_t live_bytes;            /* live_bytes() */
    uint64_t len;                   /* slots in use (the arena prefix) */
    uint64_t hot, warm, cold;       /* counts() */
    uint64_t nocorr;                /* nocorr_count() */
    uint64_t reclaimed_correction;  /* reclaimed_correction_bytes() */
    uint64_t log_errors;            /* log_errors() */
    uint64_t blocked_evictions;     /* blocked_evictions() */
} SlhaCcosStats;

/* ElasticKvCache::new / with_eviction (ccos.rs:131-193) over `arena_dev`
 * (capacity tiles, caller-owned, outlives the cache). sink_window is used by
 * SLHA_CCOS_EVICT_IMPORTANCE. NULL on failure (last error set). */
SlhaCcos* slha_ccos_new(SciRustSlhaTile* arena_dev, size_t capacity, size_t budget_bytes,
                        int32_t page_policy, int32_t eviction_policy, size_t sink_window);
int32_t slha_ccos_free(SlhaCcos* c);

/* attach_event_log / attach_durable_event_log (ccos.rs:151-167). The log
 * handle stays owned by the caller and must outlive the attachment; NULL
 * detaches. */
int32_t slha_ccos_attach_event_log(SlhaCcos* c, SlhaEventLog* log, int32_t durable);

/* insert (ccos.rs:213-247) of n device tiles, in order: each takes the last
 * recycled slot (free-list pop) or the next new one; its state follows its
 * FLAG_WARM; importance 0; a new seq. slots_out (host, n) receives the slots.
 * SLHA_ERR_DIMENSION when the arena is full. tiles_dev must not overlap the
 * arena's recycled slots (the copy into them is one parallel scatter). */
int32_t slha_ccos_insert(SlhaCcos* c, const SciRustSlhaTile* tiles_dev, size_t n, uint32_t* slots_out,
                         void* stream);

/* observe_scores (ccos.rs:257-300) for the scores of every slot of the arena
 * prefix: scores_dev[s] for s < len (e.g. slha_gpu_score over the first len
 * tiles). COLD slots are skipped; a non-finite live score, a non-finite or
 * non-positive temperature, or no live slot leaves importance unchanged.
 * Importance[s] += softmax((score - max) / temperature)[s] in f32; the sum is
 * a tree sum, so the result is within a few ulps of the reference's.
 * Returns once the kernels are enqueued on `stream` (no synchronisation);
 * scores_dev must stay valid until they run. */
int32_t slha_ccos_observe_scores(SlhaCcos* c, const float* scores_dev, size_t n, float temperature,
                                 void* stream);

/* enforce_budget (ccos.rs:519-614): drop HOT correction planes, page
 * HOT->WARM, drop WARM correction planes, then evict per the eviction policy,
 * each phase in its order and only while over budget. *within_out = 1 when
 * the footprint ends within the budget. */
int32_t slha_ccos_enforce_budget(SlhaCcos* c, int32_t* within_out, void* stream);

/* page_out / drop_correction / evict of one slot (ccos.rs:369-438); *done_out
 * says whether the slot changed (evict: whether it became COLD). */
int32_t slha_ccos_page_out(SlhaCcos* c, uint32_t slot, void* stream);
int32_t slha_ccos_drop_correction(SlhaCcos* c, uint32_t slot, int32_t* done_out, void* stream);
int32_t slha_ccos_evict(SlhaCcos* c, uint32_t slot, int32_t* done_out, void* stream);

/* rehydrate (ccos.rs:451-466): the latest record with `seq` in the attached
 * log is inserted again (new slot, new seq, importance 0). *slot_out = -1
 * when no log is attached or no record matches. */
int32_t slha_ccos_rehydrate(SlhaCcos* c, uint64_t seq, int64_t* slot_out, void* stream);

int32_t slha_ccos_stats(const SlhaCcos* c, SlhaCcosStats* out);

/* Host copies of the per-slot control state for slots [0, n), n <= len:
 * state (SLHA_CCOS_*), seq, importance. Any output may be NULL. */
int32_t slha_ccos_slots(SlhaCcos* c, size_t n, int32_t* state_out, uint64_t* seq_out,
                        float* importance_out, void* stream);

#ifdef __cplusplus
}
#endif
#endif
