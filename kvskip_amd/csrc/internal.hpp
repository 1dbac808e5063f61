// Launch-side declarations shared between the C ABI (capi.hip) and the kernel files.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kvskip_amd.h"

namespace kvs {

// Kernel argument block of the attention kernels: the validated C-ABI arguments plus the
// derived constants the kernels use (log2-domain scale, nb, log2 tau, P row length).
struct AttnP {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t q_sb, q_sh;
  int64_t k_sb, k_sh, k_st;
  int64_t v_sb, v_sh, v_st;
  int B, Hq, Hkv, T, nb;
  float scale_log2;
  const int* block_idx;
  const int* block_cnt;
  int max_blocks;
  int num_splits;
  float* part_acc;
  float* part_ml;
  uint16_t* out;
  float* out_f32;
  float* lse;
  float* blk_max;
  float* blk_sum;
  uint16_t* p_out;
  const uint16_t* p_in;
  const float* blk_scale;
  int64_t t_pad;
  float log2_tau;
  int local;
  int* vcount;
  const float* lse_prev;
  const int* seq_lens;  // [B] or null: sequence b uses tokens [0, clamp(seq_lens[b], 1, T))
  const int* block_table;  // [B, bt_stride] or null: paged K / V (page stride k_sb / v_sb)
  int64_t bt_stride;
  int num_pages;
  uint8_t* v_keep;  // single-pass V-skip: [B, Hkv, nb] 1 where the block's V was read
  int list_partition;  // masked ragged pass: 0 per KV head, 1 over all B * Hkv lists
};

// The planned pass's argument segment (AttnP, kvskip_plan_args and, where an update is carried,
// kvskip_update_args: 640 or 808 bytes, 10 or 13 lines of 64 bytes) loaded into the scalar cache
// in one batch with one wait, as the kernel's first statement (the loaded words are unused). Read
// where the code first needs each field, the compiler waited for its lines in two or three rounds
// before the first list and K / V loads (per layer-step, 64 steps: config 4's loop 36.47 -> 36.08
// us, the refresh mode's two planned passes 46.78 -> 46.10). The
// segment holds 256 bytes of hidden arguments after the explicit ones, so no line read lies outside.
#define KVS_KL(i, off) "s_load_dword %" #i ", %[kp], " #off "\n\t"
template <bool UPDATE>
__device__ __forceinline__ void prefetch_planned_args() {
  const auto kp = __builtin_amdgcn_kernarg_segment_ptr();
  uint32_t d0, d1, d2, d3, d4, d5, d6, d7, d8, d9, d10, d11, d12;
  if constexpr (UPDATE) {
    asm volatile(KVS_KL(0, 0x0) KVS_KL(1, 0x40) KVS_KL(2, 0x80) KVS_KL(3, 0xc0) KVS_KL(4, 0x100)
                 KVS_KL(5, 0x140) KVS_KL(6, 0x180) KVS_KL(7, 0x1c0) KVS_KL(8, 0x200) KVS_KL(9, 0x240)
                 KVS_KL(10, 0x280) KVS_KL(11, 0x2c0) KVS_KL(12, 0x300) "s_waitcnt lgkmcnt(0)"
                 : "=&s"(d0), "=&s"(d1), "=&s"(d2), "=&s"(d3), "=&s"(d4), "=&s"(d5), "=&s"(d6), "=&s"(d7),
                   "=&s"(d8), "=&s"(d9), "=&s"(d10), "=&s"(d11), "=&s"(d12)
                 : [kp] "s"(kp) : "memory");
  } else {
    asm volatile(KVS_KL(0, 0x0) KVS_KL(1, 0x40) KVS_KL(2, 0x80) KVS_KL(3, 0xc0) KVS_KL(4, 0x100)
                 KVS_KL(5, 0x140) KVS_KL(6, 0x180) KVS_KL(7, 0x1c0) KVS_KL(8, 0x200) KVS_KL(9, 0x240)
                 "s_waitcnt lgkmcnt(0)"
                 : "=&s"(d0), "=&s"(d1), "=&s"(d2), "=&s"(d3), "=&s"(d4), "=&s"(d5), "=&s"(d6), "=&s"(d7),
                   "=&s"(d8), "=&s"(d9)
                 : [kp] "s"(kp) : "memory");
  }
}
#undef KVS_KL
static_assert(sizeof(AttnP) + sizeof(kvskip_plan_args) == 640 && sizeof(kvskip_update_args) == 168,
              "the planned pass's argument lines");

constexpr int MAX_RAGGED_B = 256;  // batch bound of the ragged partition (one scan per 64)
constexpr int MAX_GLOBAL_LISTS = 512;  // B * Hkv bound of the partition over all lists

constexpr int MAX_SPLITS = 256;

// QK engine of the attention kernels: MFMA (default) unless KVSKIP_AMD_QK=valu.
bool qk_use_mfma();

// Head dims / group sizes with instantiated attention kernels.
bool attn_supported(int D, int G);

// Each returns a hipError_t of the launch(es).
// launch_decode phase: bit 0 the split pass, bit 1 the split merge (3: both, as one op).
hipError_t launch_decode(const AttnP& p, int D, int G, bool masked, bool stats, bool load_v, int phase,
                         hipStream_t s);
// launch_decode over a paged cache (p.block_table set; the MFMA engine), same phases.
hipError_t launch_decode_paged(const AttnP& p, int D, int G, bool masked, bool stats, bool load_v, int phase,
                               hipStream_t s);
hipError_t launch_vskip1(const AttnP& p, int D, int G, hipStream_t s);
hipError_t launch_pv(const AttnP& p, int D, int G, hipStream_t s);
// Two-pass V-skip pass 2 with the selection of sel in its prologue (then its split merge).
hipError_t launch_pv_select(const AttnP& p, const kvskip_select_args& sel, int D, int G, hipStream_t s);
hipError_t launch_read(const void* x, int64_t bytes, uint32_t* out, int blocks, hipStream_t s);

hipError_t launch_plan(const kvskip_plan_args& p, hipStream_t s);
hipError_t launch_update(const kvskip_update_args& p, hipStream_t s);
// The split merge of an attention pass (num_splits >= 2, with V) and a planner update, one launch.
hipError_t launch_merge_update(const AttnP& a, const kvskip_update_args& p, int D, hipStream_t s);
// The masked + statistics split pass of a (phase 1) and the update u of another layer, one launch.
hipError_t launch_split_update(const AttnP& a, const kvskip_update_args& u, int D, hipStream_t s);
// launch_split_update's fused form over a paged cache (its own translation unit).
hipError_t launch_split_update_paged(const AttnP& a, const kvskip_update_args& u, int D, hipStream_t s);
// The plan's decision + the masked statistics split pass of a (phase 1) in one launch, with an
// optional carried update u of another layer.
hipError_t launch_planned_split(const AttnP& a, const kvskip_plan_args& pa, const kvskip_update_args* u, int D,
                                hipStream_t s);
// launch_planned_split over a paged cache, after any unfused carried update (its own translation
// unit).
hipError_t launch_planned_paged(const AttnP& a, const kvskip_plan_args& pa, const kvskip_update_args* u, int D,
                                hipStream_t s);
// launch_planned_split over a ragged batch (seq_lens, B > 1) of a contiguous cache, after any
// unfused carried update (its own translation unit).
hipError_t launch_planned_ragged(const AttnP& a, const kvskip_plan_args& pa, const kvskip_update_args* u, int D,
                                 hipStream_t s);
// The plan's first launch alone (the scores pass; needs part).
hipError_t launch_plan_scores(const kvskip_plan_args& p, hipStream_t s);
hipError_t launch_block_sums(const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st, int B, int Hkv, int T,
                             int D, float* csum, int NBC, const int32_t* seq_lens, const int32_t* tbl, int64_t bt,
                             int npages, hipStream_t s);
hipError_t launch_token_index(const int32_t* ids, int64_t ids_stride, int B, int T, uint8_t* idx, int NBC,
                              const int32_t* seq_lens, hipStream_t s);

// Block selection (select.hip): the GQA-union rule, list and scales; the list of a keep mask.
hipError_t launch_select(const kvskip_select_args& a, hipStream_t s);
hipError_t launch_block_list(const uint8_t* keep, int B, int Hkv, int nb, int32_t* block_idx, int32_t* block_cnt,
                             hipStream_t s);

// Largest block count the planner kernels hold in LDS for a group of G query heads.
int planner_max_blocks(int G);
int64_t plan_part_floats(int B, int Hq, int Hkv, int NBC);

}  // namespace kvs
