/*
 * kvskip_amd: C ABI of the MI355X (gfx950) decode-attention hot path.
 *
 * Every entry point takes plain pointers to device memory, element strides and sizes,
 * and a HIP stream (hipStream_t passed as void*; NULL = the null stream). Nothing is
 * allocated inside the library: outputs and split-K partial buffers are passed in by the
 * caller. Entry points validate their arguments on the host before any device work and
 * return KVSKIP_OK (0) or a negative KVSKIP_E* code; kvskip_last_error() then holds a
 * message for the calling thread. No entry point synchronises with the host.
 *
 * Units. Scores are q.k * scale. blk_max and lse are natural-log units; the split-K
 * partials (part_ml) are in log2 units (running max, running sum), as are all internal
 * softmax states. Blocks are 64 tokens from position 0; nb = ceil(T / 64).
 *
 * Each entry point names the reference interface it replaces (format37/kvskip, paths
 * relative to its repository root).
 */
#ifndef KVSKIP_AMD_H
#define KVSKIP_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KVSKIP_BLOCK 64

enum {
  KVSKIP_OK = 0,
  KVSKIP_E_INVALID = -1,     /* argument validation failed (message in kvskip_last_error) */
  KVSKIP_E_UNSUPPORTED = -2, /* head dim / group size / flag combination not instantiated */
  KVSKIP_E_LAUNCH = -3       /* the HIP runtime rejected a launch */
};

/* Attention launch block: replaces kvskip::Params (kernels/kvskip.h:13-60).
 * q [B, Hq, D] bf16; k, v [B, Hkv, T, D] bf16 with arbitrary batch/head/token element
 * strides, D contiguous, all strides multiples of 8 elements, base 16-byte aligned. */
typedef struct kvskip_attn_args {
  const void* q;
  const void* k;
  const void* v;
  int64_t q_sb, q_sh;
  int64_t k_sb, k_sh, k_st;
  int64_t v_sb, v_sh, v_st;
  int32_t B, Hq, Hkv, T, D;
  float scale;                 /* softmax scale (natural units) */

  /* masked mode: per (b, kv head) ascending list of block indices to read */
  const int32_t* block_idx;    /* [B, Hkv, max_blocks] */
  const int32_t* block_cnt;    /* [B, Hkv] */
  int32_t max_blocks;

  /* split-K: num_splits > 1 needs both partial buffers */
  int32_t num_splits;
  float* part_acc;             /* [B, Hq, num_splits, D] un-normalised, relative to the part max */
  float* part_ml;              /* [B, Hq, num_splits, 2] (max, sum) in log2 units */

  void* out;                   /* [B, Hq, D] bf16 (NULL in stats-only mode) */
  float* out_f32;              /* optional [B, Hq, D] */
  float* lse;                  /* optional [B, Hq] natural-log log-sum-exp of the attended scores */

  /* per-block statistics, [B, Hq, nb]: max score (natural units) and sum exp(s - max);
   * every block is written, (-inf, 0) where the list skips it (the reference leaves those to a
   * host-side fill, kernels/kvskip_ext.cpp:51-54; here the masked pass writes them) */
  float* blk_max;
  float* blk_sum;

  /* two-pass V-skip: pass 1 writes P = exp(s - blk_max) as fp16 [B, Hq, nb*64];
   * pass 2 reads it back with blk_scale [B, Hkv, nb, G] */
  void* p_out;
  const void* p_in;
  const float* blk_scale;

  /* single-pass V-skip */
  float tau;                   /* keep V of a block if some head's weight estimate >= tau */
  int32_t local;               /* newest blocks always kept (block 0 always kept too) */
  int32_t* vcount;             /* optional [B, Hkv] V blocks loaded (atomically added) */
  const float* lse_prev;       /* optional [B, Hq] natural-log normaliser estimate; NULL: block-0 bound */

  /* Ragged batch (not in the reference; kvskip_decode only): optional [B] int32 device array,
   * sequence b attends tokens [0, clamp(seq_lens[b], 1, T)) of its view (T = the views' capacity,
   * nb = ceil(T / 64) sizes the statistics). The split pass then partitions each KV head's work
   * over the whole batch: chunks of C = ceil(sum_b items_b / num_splits) blocks (or list entries),
   * so every workgroup gets at most C whatever the lengths; needs num_splits >= 2, B <= 256, and
   * part_acc / part_ml of [B, Hq, num_splits, ...]. */
  const int32_t* seq_lens;

  /* Paged cache (not in the reference; every pass that reads K or V: kvskip_decode and its split
   * entry points, kvskip_pv, kvskip_vskip1; MFMA engine; at most 4096 blocks per split): k and v
   * point to page pools of 64-token pages; token t of sequence b, KV head h
   * is row t % 64 of page block_table[b * bt_stride + t / 64], at k + page * k_sb + h * k_sh +
   * (t % 64) * k_st (k_sb, v_sb: the page stride). T is the sequences' length (or capacity with
   * seq_lens); bt_stride >= ceil(T / 64). A page id outside [0, num_pages) makes its block empty
   * (scores -inf, statistics (-inf, 0)); no memory outside the pools is read. */
  const int32_t* block_table;
  int64_t bt_stride;
  int32_t num_pages;

  /* Single-pass V-skip (not in the reference, which reports only vcount): optional
   * [B, Hkv, ceil(T / 64)] uint8, 1 where the block's V was read (entered the softmax), else 0. */
  uint8_t* v_keep;

  /* Partition of a masked ragged pass (not in the reference; block_idx with seq_lens): 0 cuts each
   * KV head's lists over the batch (chunks of ceil(sum_b cnt / num_splits) entries per head); 1
   * cuts all B * Hkv lists by one length C = max(ceil(sum / (num_splits * Hkv)), ceil(max cnt /
   * num_splits)), so a KV head whose lists hold more entries gets more workgroups (needs
   * B * Hkv <= 512). The merge (kvskip_merge_splits) must be given the value its pass had. */
  int32_t list_partition;
} kvskip_attn_args;

/* Split-K decode attention: dense (block_idx NULL) or over block lists, with optional per-block
 * statistics (stats), stats-only reading K alone (load_v = 0, needs stats) and fp16 P (p_out,
 * needs stats). num_splits (1..256) > 1 adds the log-sum-exp merge of the partials.
 * Replaces kvskip::launch_decode (kernels/kvskip.h:113-114, kernels/kvskip_kernel.cu:761-769),
 * reached from kvskip_ext.decode (kernels/kvskip_ext.cpp:25-101). Any G = Hq / Hkv in 1..8. */
int kvskip_decode(const kvskip_attn_args* a, int stats, int load_v, void* stream);

/* kvskip_decode as its two launches (num_splits >= 2; same arguments, called in this order on
 * one stream): the split pass into part_acc / part_ml (+ statistics), then the split merge into
 * out / out_f32 / lse. Not in the reference (its launch_decode issues both,
 * kernels/kvskip_kernel.cu:433-473): for timing each kernel on its own or scheduling other work
 * between the two. */
int kvskip_decode_splits(const kvskip_attn_args* a, int stats, int load_v, void* stream);
int kvskip_merge_splits(const kvskip_attn_args* a, int stats, int load_v, void* stream);

/* kvskip_decode without caller-provided split partials: no counterpart in the reference. For
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). a->part_acc and a->part_ml are ignored; the split-K partials
 * go to a library-owned static device array of KVSKIP_SCRATCH_BYTES per GPU, so
 * B * Hq * num_splits * (D + 2) * 4 bytes (plus alignment) must fit, else KVSKIP_E_INVALID. Every
 * other argument, and the results, as kvskip_decode. Nothing is allocated or freed. All calls on
 * one GPU share its array: calls that overlap in time on one GPU (two streams, two threads) race. */
#define KVSKIP_SCRATCH_BYTES (16LL << 20)
int kvskip_decode_scratch(const kvskip_attn_args* a, int stats, int load_v, void* stream);

/* Two-pass V-skip, pass 2: out = sum over listed blocks of blk_scale * P . V (no softmax);
 * num_splits > 1 adds the plain sum of the partials.
 * Replaces kvskip::launch_pv (kernels/kvskip.h:117, kernels/kvskip_kernel.cu:754-759),
 * reached from kvskip_ext.pv (kernels/kvskip_ext.cpp:106-146). */
int kvskip_pv(const kvskip_attn_args* a, void* stream);

/* Single-pass V-skip: every K block is read; the V block is read (and the block enters the
 * softmax) only for block 0, the `local` newest blocks, or when some head of the group has
 * block log-sum-exp - lse0 >= log(tau), lse0 = lse_prev or the block-0 log-sum-exp.
 * Replaces kvskip::launch_vskip1 (kernels/kvskip.h:118, kernels/kvskip_kernel.cu:747-752),
 * reached from kvskip_ext.vskip1 (kernels/kvskip_ext.cpp:149-195). */
int kvskip_vskip1(const kvskip_attn_args* a, void* stream);

/* Streaming read of `bytes` (multiple of 16) bytes at x: the achievable read ceiling.
 * Replaces kvskip::launch_read (kernels/kvskip.h:120), kvskip_ext.read_bw
 * (kernels/kvskip_ext.cpp:321-325). out: one uint32 (written only if a sentinel hits). */
int kvskip_read(const void* x, int64_t bytes, uint32_t* out, int32_t blocks, void* stream);

/* Refresh planner, before the attention pass. Replaces kvskip::PlanParams + launch_plan
 * (kernels/kvskip.h:63-89,115, kernels/kvskip_planner.cu:75-227,309-312), reached from
 * kvskip_ext.plan (kernels/kvskip_ext.cpp:205-267). Any D in {64, 128}, G in 1..8. */
typedef struct kvskip_plan_args {
  const void* q;               /* [B, Hq, D] bf16 */
  int64_t q_sb, q_sh;
  const void* k;               /* [B, Hkv, T, D] bf16 cache view, the new token at T - 1 */
  int64_t k_sb, k_sh, k_st;
  float* csum;                 /* [B, Hkv, NBC, D] per-block key sums (fp32), updated if add_token */
  const float* lse_ref;        /* [B, Hq, NBC] block log-sum-exp at the head's last refresh */
  const float* cs_ref;         /* [B, Hq, NBC] centroid scores at that refresh */
  const uint8_t* keep;         /* [B, Hkv, NBC] stored set */
  const float* lse_att;        /* [B, Hq] previous step's attended log-sum-exp */
  int32_t* age;                /* [B, Hkv] steps since the last refresh (updated) */
  const int32_t* flags;        /* [Hkv] bit 0 always refresh, bit 1 token-index head, bit 2 index union */
  const uint8_t* idx;          /* [B, NBC] token-index blocks, or NULL */
  const float* calib;          /* [B, Hkv] estimate correction, or NULL */
  float* est;                  /* [B, Hkv] out: uncorrected estimate, or NULL */
  const uint8_t* aix;          /* [B, Hkv] heads latched onto the index, or NULL (needs idx) */
  float* cs_now;               /* [B, Hq, NBC] out: this step's centroid scores */
  uint8_t* trig;               /* [B, Hkv] out: refresh decision */
  int32_t* block_idx;          /* [B, Hkv, NBC] out: blocks to read, ascending */
  int32_t* block_cnt;          /* [B, Hkv] out */
  int32_t B, Hq, Hkv, T, D, NBC, local, max_age, add_token, calib_on, calib_kind;
  float scale, delta;
  /* Optional workspace (not in the reference): >= kvskip_plan_part_floats(B, Hq, Hkv, NBC)
   * floats. With it the centroid pass runs on ceil(nb / 32) workgroups per head and a second
   * launch decides and compacts; NULL: one workgroup per head, one launch. Calls sharing a
   * workspace must not overlap. */
  float* part;
  /* Optional [B] int32 device array (not in the reference): ragged batch, sequence b holds
   * clamp(seq_lens[b], 1, T) tokens (T = the views' capacity); add_token adds each sequence's
   * last row. */
  const int32_t* seq_lens;
  /* Optional [B] int32 device array (not in the reference): the plan writes each sequence's
   * length (clamp(seq_lens[b], 1, T), or T) here, so that the update of the same step can read
   * the lengths from memory that only the next plan rewrites (the device planner loop hands a
   * layer's update to a later launch). */
  int32_t* seq_lens_out;
  /* Optional, with part (not in the reference): token ids [B, >= T] int32, row stride ids_sb
   * elements. The plan then finds this step's token-index blocks itself (kvskip_token_index's
   * rule), uses them as idx (which must be NULL) and writes them to idx_out [B, NBC] for the
   * update (blocks >= ceil(T / 64): untouched). One launch fewer per layer-step. */
  const int32_t* ids;
  int64_t ids_sb;
  uint8_t* idx_out;
  /* Optional paged cache for the appended key row (not in the reference), as in kvskip_attn_args:
   * k a page pool, k_sb its page stride; an invalid page leaves the key sums as they are. */
  const int32_t* block_table;
  int64_t bt_stride;
  int32_t num_pages;
  /* Optional, read by kvskip_decode_splits_planned only (not in the reference): 0, or the pass's
   * workgroup budget over all B * Hkv (<= 16) lists together. Every workgroup then decides all the
   * lists and cuts them into chunks of one length over all of them (a refreshing head gets more
   * workgroups than a light one); the pass's num_splits is the count of split-partial slots per
   * head (each list gets at most that many chunks), and the slots a list leaves unused are written
   * empty, so the split merge takes num_splits as usual. The grid is pass_budget + B * Hkv
   * workgroups. */
  int32_t pass_budget;
  /* Read by kvskip_decode_splits_planned only (not in the reference): the decision the pass makes.
   *   KVSKIP_DECIDE_PLAN (0)  plan's: the refreshing heads read every block, the others their
   *                           attended set (stored set + block 0 + the `local` newest).
   *   KVSKIP_DECIDE_LISTS     no decision: every head reads its attended set; trig and est are not
   *                           written.
   *   KVSKIP_DECIDE_POST      the decision against the log-sum-exp of this step's LISTS pass
   *                           (lse_part below, or lse_att): a refreshing head reads the blocks
   *                           OUTSIDE its attended set, the others nothing, and no (-inf, 0)
   *                           statistics are written for unlisted blocks (the LISTS pass wrote the
   *                           attended blocks' statistics and (-inf, 0) for the rest; a refreshing
   *                           head's rest comes from this pass). The lists written are these.
   * LISTS into partial slots [0, S), then POST into [S, 2S), then one split merge over the 2S slots
   * is the reference's "refresh" mode (src/kvskip_attn.py:233-270: attention over the stored sets,
   * the estimate and trigger against that pass's lse, attention and statistics over every block
   * for the refreshing heads, whose outputs replace the masked ones): a refreshing head's merge
   * joins its attended and its other blocks, every block read once. */
  int32_t decide_mode;
  /* Read by kvskip_decode_splits_planned only (not in the reference): the pass's partials go to slots
   * [slot_base, slot_base + slot_count) of each query head's num_splits slots (slot_count 0: all
   * num_splits from 0), and a list gets at most slot_count chunks. */
  int32_t slot_base, slot_count;
  /* Read by the POST decision only (not in the reference): if not NULL, the attended log-sum-exp
   * comes from the split partials of the step's LISTS pass instead of lse_att: lse_part is that
   * pass's part_ml ([B, Hq, lse_stride, 2], max and sum in log2 units), slots [0, lse_slots)
   * (lse_slots <= 64). */
  const float* lse_part;
  int32_t lse_slots, lse_stride;
  /* Optional, with part (not in the reference): [B * Hkv] int32, zero before the first call and left
   * zero by every call. kvskip_plan is then ONE launch: the last scores workgroup of each (b, KV
   * head) to finish (counted on its ticket with an agent-scope atomic, after agent-scope stores of
   * the partials) makes the head's decision and writes its list. Calls that share a ticket array
   * must not overlap in time. Ignored by kvskip_plan_scores and kvskip_decode_splits_planned. */
  int32_t* ticket;
} kvskip_plan_args;

#define KVSKIP_DECIDE_PLAN 0
#define KVSKIP_DECIDE_LISTS 1
#define KVSKIP_DECIDE_POST 2

int kvskip_plan(const kvskip_plan_args* p, void* stream);

/* The first launch of kvskip_plan with a workspace alone: the scores pass (needs part). Not in the
 * reference: with kvskip_decode_splits_planned after it, the decision runs inside the masked pass. */
int kvskip_plan_scores(const kvskip_plan_args* p, void* stream);

/* Floats of kvskip_plan_args.part for a state of capacity NBC blocks (-1 for invalid sizes).
 * Not in the reference: sizes the optional multi-workgroup plan workspace. */
int64_t kvskip_plan_part_floats(int32_t B, int32_t Hq, int32_t Hkv, int32_t NBC);

/* Refresh planner, after the attention pass. Replaces kvskip::UpdateParams + launch_update
 * (kernels/kvskip.h:91-111,116, kernels/kvskip_planner.cu:229-305,314-318), reached from
 * kvskip_ext.update (kernels/kvskip_ext.cpp:270-319). */
typedef struct kvskip_update_args {
  const float* blk_max;        /* [B, Hq, nb] stats of this step's pass (-inf / 0 where not read) */
  const float* blk_sum;
  const uint8_t* trig;         /* [B, Hkv] */
  const float* cs_now;         /* [B, Hq, NBC] */
  uint8_t* keep;               /* [B, Hkv, NBC] updated on refreshing heads */
  float* lse_ref;              /* [B, Hq, NBC] updated on refreshing heads */
  float* cs_ref;               /* [B, Hq, NBC] updated on refreshing heads */
  float* lse_att;              /* [B, Hq] updated on every head */
  const int32_t* flags;        /* [Hkv] or NULL */
  const uint8_t* idx;          /* [B, NBC] or NULL */
  const float* est;            /* [B, Hkv] plan's uncorrected estimate (with calib) */
  float* calib;                /* [B, Hkv] or NULL: no learning */
  uint8_t* aix;                /* [B, Hkv] or NULL */
  float calib_rate, aix_thr, level;
  int32_t calib_free, calib_kind;
  int32_t B, Hq, Hkv, T, NBC, local;
  int32_t list_stats;          /* 0: blk_max / blk_sum cover every block (the reference's contract);
                                  1: they hold values only for the blocks of this step's plan (the
                                  rest is uninitialised and ignored), so they need no fill */
  const int32_t* seq_lens;     /* optional [B] int32 (ragged batch, as in kvskip_plan_args); the
                                  statistics keep the row length ceil(T / 64) */
  int32_t* age;                /* optional [B, Hkv] (not in the reference): the plan's age, advanced
                                  here (0 if trig, else + 1; token-index heads untouched) when the
                                  decision ran in the pass (kvskip_decode_splits_planned) */
} kvskip_update_args;

int kvskip_update(const kvskip_update_args* p, void* stream);

/* kvskip_merge_splits of an attention pass (num_splits >= 2, load_v) and kvskip_update of the
 * planner in one launch (disjoint workgroups: both read only what the split pass wrote). Not in
 * the reference: the device planner loop's pass ends this way (kvskip_decode_splits, then this). */
int kvskip_merge_update(const kvskip_attn_args* a, const kvskip_update_args* u, void* stream);

/* kvskip_decode_splits of a masked + statistics pass (block list, stats, load_v; with
 * num_splits == 1 the whole op) and kvskip_update u of ANOTHER layer, in one launch. Not in the
 * reference: a layer's update only reads that layer's statistics and is only read by that
 * layer's next plan, so the device planner loop runs it inside the next layer's pass (under its
 * streaming) instead of in a launch of its own. u and a must not share outputs; u's group size
 * equals a's. Updates over more than 1536 blocks, or with the VALU engine selected, run as two
 * launches (same results). */
int kvskip_decode_splits_update(const kvskip_attn_args* a, const kvskip_update_args* u, void* stream);

/* The second half of kvskip_plan and the masked + statistics split pass in one launch (not in the
 * reference): after kvskip_plan_scores(p), every workgroup of the pass merges the partials of its
 * (b, KV head), makes plan's decision (the same result in every workgroup) and takes its slice of
 * the block list from the attended-block masks; p's trig, est, block_idx and block_cnt are written
 * as by kvskip_plan, but NOT the age: the layer's update must advance it (u->age). a: as for
 * kvskip_decode_splits with stats and load_v (its block list fields are ignored); seq_lens, the same
 * array in a and p: with B == 1 the step's length in device memory; with 1 < B <= 16 a ragged batch
 * of a contiguous cache (the ragged grid and partition of kvskip_decode_splits, cut over the lists
 * the workgroups decide; then pass_budget, slot_base, slot_count are 0, lse_part NULL and decide_mode
 * PLAN or LISTS; its merge is kvskip_merge_splits with the same seq_lens and lists).
 * u: NULL, or the update of another layer to carry (as kvskip_decode_splits_update). */
int kvskip_decode_splits_planned(const kvskip_attn_args* a, const kvskip_plan_args* p, const kvskip_update_args* u,
                                 void* stream);

/* Per-block key sums of the first T tokens: csum[b, h, blk, :] = sum of k rows of the block
 * (fp32), blocks >= nb up to NBC zeroed. The device form of _centroid_sums
 * (src/kvskip_attn.py:170-179), used to initialise the planner state on the device. seq_lens: optional
 * [B] int32 device array (ragged batch: sequence b sums its first clamp(seq_lens[b], 1, T) rows).
 * block_table, bt_stride, num_pages: optional paged cache, as in kvskip_attn_args (k a page pool,
 * k_sb its page stride); a block on an invalid page sums to zero. */
int kvskip_block_sums(const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st, int32_t B, int32_t Hkv,
                      int32_t T, int32_t D, float* csum, int32_t NBC, const int32_t* seq_lens,
                      const int32_t* block_table, int64_t bt_stride, int32_t num_pages, void* stream);

/* Token index of a decode step: idx[b, blk] = 1 if block blk (of the first T tokens) holds an
 * earlier copy of ids[b, T-1] or the position right after one; blocks >= nb up to NBC are
 * zeroed. The device form of index_steps / index_blocks (src/lab.py:149-167,
 * src/run_free.py:103-113). ids [B, ids_stride] int32. seq_lens: optional [B] int32 device array
 * (ragged batch: sequence b's current token is ids[b, clamp(seq_lens[b], 1, T) - 1]). */
int kvskip_token_index(const int32_t* ids, int64_t ids_stride, int32_t B, int32_t T, uint8_t* idx,
                       int32_t NBC, const int32_t* seq_lens, void* stream);

/* GQA-union block selection from per-block statistics, on the device. Replaces the torch steps of
 * the reference's two-pass V-skip between its passes: select_blocks (kernels/kvskip.py:130-147),
 * the kept-set normaliser and per-block scales (kernels/kvskip.py:168-172) and make_plan's list
 * (kernels/kvskip.py:79-85). Per query head the block log-weights x = blk_max + log blk_sum
 * (-inf where blk_sum is 0); rule 0 ("tau") keeps blocks with softmax weight >= value, rule 1
 * ("topp") the fewest blocks whose weights reach value (ties at the cut kept); a KV head keeps the
 * union over its G query heads plus block 0 and the `local` newest. Every output is optional. */
typedef struct kvskip_select_args {
  const float* blk_max;        /* [B, Hq, nb] */
  const float* blk_sum;        /* [B, Hq, nb] */
  int32_t B, Hq, Hkv, nb;      /* G = Hq / Hkv <= 8, nb <= 4096 */
  int32_t rule;                /* 0 tau, 1 topp */
  float value;                 /* tau, or the top-p level */
  int32_t local;
  uint8_t* keep;               /* out [B, Hkv, nb]: 1 kept, 0 not */
  int32_t* block_idx;          /* out [B, Hkv, nb]: kept blocks ascending, then the others ascending */
  int32_t* block_cnt;          /* out [B, Hkv] (with block_idx) */
  float* blk_scale;            /* out [B, Hkv, nb, G]: exp(blk_max - lse over the kept blocks), 0 off the set */
} kvskip_select_args;

int kvskip_select(const kvskip_select_args* s, void* stream);

/* Two-pass V-skip pass 2 with the selection in it (not in the reference, which selects with torch
 * ops between its two decode calls, kernels/kvskip.py:157-179): kvskip_select(s) followed by
 * kvskip_pv(a) over the lists and scales it writes, in one launch (+ the split merge): every
 * workgroup of the pass makes its (b, KV head)'s selection, takes its split of the kept blocks
 * (ascending) and computes their scales. Same results bit for bit. a: as for kvskip_pv without
 * block_idx / block_cnt / blk_scale (contiguous cache, no seq_lens); s: the selection, over the
 * same B, Hq, Hkv and nb; its outputs (keep, block_idx / block_cnt, blk_scale) are optional. */
int kvskip_pv_select(const kvskip_attn_args* a, const kvskip_select_args* s, void* stream);

/* The kept-first block list of a keep mask keep [B, Hkv, nb] (uint8, nonzero = kept): block_idx
 * [B, Hkv, nb] the kept blocks ascending then the others ascending, block_cnt [B, Hkv]. The device
 * form of make_plan (kernels/kvskip.py:79-85, a stable argsort of ~keep). */
int kvskip_block_list(const uint8_t* keep, int32_t B, int32_t Hkv, int32_t nb, int32_t* block_idx,
                      int32_t* block_cnt, void* stream);

/* Message of the last failed call on this thread ("" if none). */
const char* kvskip_last_error(void);

/* Library version string. */
const char* kvskip_version(void);

/* sizeof of the argument blocks (0: kvskip_attn_args, 1: kvskip_plan_args, 2: kvskip_update_args,
 * 3: kvskip_select_args), -1 otherwise: lets a binding check its struct layout. Library utility, no
 * reference counterpart. */
int kvskip_struct_size(int which);

#ifdef __cplusplus
}
#endif

#endif /* KVSKIP_AMD_H */
