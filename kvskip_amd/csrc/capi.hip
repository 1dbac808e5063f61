// C ABI of kvskip_amd: host-side argument validation, derived launch constants, launches.
// Validation never touches the device, so every error path runs without a GPU.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "internal.hpp"

namespace {

// Split-K partials of kvskip_decode_scratch: library-owned device memory, one copy per GPU (each
// device that loads the library holds it until the process ends). Host code must never use this
// name as an address: kvskip_decode_scratch takes each device's address from hipGetSymbolAddress.
constexpr int64_t SCRATCH_FLOATS = KVSKIP_SCRATCH_BYTES / 4;
__device__ __align__(256) float scratch[SCRATCH_FLOATS];

constexpr int SCRATCH_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[SCRATCH_MAX_DEVICES] = {};

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return KVSKIP_OK;
}

int launched(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(KVSKIP_E_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return ok();
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_kv(const void* ptr, int64_t sb, int64_t sh, int64_t st, const char* name) {
  if (ptr == nullptr) return fail(KVSKIP_E_INVALID, "%s must be a CUDA bf16 tensor", name);
  if (sb % 8 != 0 || sh % 8 != 0 || st % 8 != 0)
    return fail(KVSKIP_E_INVALID, "%s strides must be multiples of 8 elements (16-byte rows)", name);
  if (!aligned16(ptr)) return fail(KVSKIP_E_INVALID, "%s must be 16-byte aligned", name);
  return KVSKIP_OK;
}

// Common checks of q/k/v and sizes; fills the derived parts of the kernel block.
int prepare_attn(const kvskip_attn_args* a, bool need_q, bool need_k, bool need_v, kvs::AttnP* p) {
  if (a == nullptr) return fail(KVSKIP_E_INVALID, "null argument block");
  if (a->B < 1 || a->Hq < 1 || a->Hkv < 1 || a->T < 1)
    return fail(KVSKIP_E_INVALID, "sizes must be positive (B=%d Hq=%d Hkv=%d T=%d)", a->B, a->Hq, a->Hkv, a->T);
  if (a->Hq % a->Hkv != 0) return fail(KVSKIP_E_INVALID, "Hq must be a multiple of Hkv");
  const int G = a->Hq / a->Hkv;
  if (!kvs::attn_supported(a->D, G))
    return fail(KVSKIP_E_UNSUPPORTED, "kvskip: unsupported head dim / group size (D=%d, G=%d)", a->D, G);
  if (need_q) {
    if (a->q == nullptr) return fail(KVSKIP_E_INVALID, "q must be CUDA bf16 [B, Hq, D]");
    if (a->q_sb % 8 != 0 || a->q_sh % 8 != 0 || !aligned16(a->q))
      return fail(KVSKIP_E_INVALID, "q rows must be 16-byte aligned");
  }
  int rc;
  if (need_k && (rc = check_kv(a->k, a->k_sb, a->k_sh, a->k_st, "k")) != KVSKIP_OK) return rc;
  if (need_v && (rc = check_kv(a->v, a->v_sb, a->v_sh, a->v_st, "v")) != KVSKIP_OK) return rc;
  if (a->num_splits < 1) return fail(KVSKIP_E_INVALID, "num_splits >= 1");
  if (a->num_splits > kvs::MAX_SPLITS) return fail(KVSKIP_E_INVALID, "num_splits <= %d", kvs::MAX_SPLITS);
  if (a->num_splits > 1 && a->part_ml == nullptr)
    return fail(KVSKIP_E_INVALID, "num_splits > 1 needs the split partial buffers");
  std::memset(p, 0, sizeof(*p));
  p->q = static_cast<const uint16_t*>(a->q);
  p->k = static_cast<const uint16_t*>(a->k);
  p->v = static_cast<const uint16_t*>(a->v);
  p->q_sb = a->q_sb; p->q_sh = a->q_sh;
  p->k_sb = a->k_sb; p->k_sh = a->k_sh; p->k_st = a->k_st;
  p->v_sb = a->v_sb; p->v_sh = a->v_sh; p->v_st = a->v_st;
  p->B = a->B; p->Hq = a->Hq; p->Hkv = a->Hkv; p->T = a->T;
  p->nb = (a->T + KVSKIP_BLOCK - 1) / KVSKIP_BLOCK;
  p->scale_log2 = static_cast<float>(static_cast<double>(a->scale) * 1.4426950408889634);
  p->block_idx = a->block_idx;
  p->block_cnt = a->block_cnt;
  p->max_blocks = a->max_blocks;
  p->num_splits = a->num_splits;
  p->part_acc = a->part_acc;
  p->part_ml = a->part_ml;
  p->out = static_cast<uint16_t*>(a->out);
  p->out_f32 = a->out_f32;
  p->lse = a->lse;
  p->blk_max = a->blk_max;
  p->blk_sum = a->blk_sum;
  p->p_out = static_cast<uint16_t*>(a->p_out);
  p->p_in = static_cast<const uint16_t*>(a->p_in);
  p->blk_scale = a->blk_scale;
  p->t_pad = static_cast<int64_t>(p->nb) * KVSKIP_BLOCK;
  p->local = a->local;
  p->vcount = a->vcount;
  p->lse_prev = a->lse_prev;
  p->seq_lens = a->seq_lens;
  p->block_table = a->block_table;
  p->bt_stride = a->bt_stride;
  p->num_pages = a->num_pages;
  p->v_keep = a->v_keep;
  p->list_partition = a->list_partition;
  return KVSKIP_OK;
}

}  // namespace

namespace kvs {
bool qk_use_mfma() {
  const char* e = std::getenv("KVSKIP_AMD_QK");
  return !(e != nullptr && std::strcmp(e, "valu") == 0);
}
}  // namespace kvs

extern "C" {

const char* kvskip_last_error(void) { return g_err; }

const char* kvskip_version(void) { return "kvskip_amd 0.1 (gfx950)"; }

int kvskip_struct_size(int which) {
  switch (which) {
    case 0: return static_cast<int>(sizeof(kvskip_attn_args));
    case 1: return static_cast<int>(sizeof(kvskip_plan_args));
    case 2: return static_cast<int>(sizeof(kvskip_update_args));
    case 3: return static_cast<int>(sizeof(kvskip_select_args));
    default: return -1;
  }
}

// Checks of a decode launch (phase: 3 the op, 1 its split pass, 2 its merge) into *p.
// A paged cache (block_table set): the MFMA engine, a table row per sequence of >= nb pages, and at
// most MAX_NB items per workgroup (their pages are gathered into LDS); `items` per (b, head).
static int check_paged(const kvskip_attn_args* a, int nb, int64_t items) {
  if (!kvs::qk_use_mfma()) return fail(KVSKIP_E_UNSUPPORTED, "paged cache: MFMA engine only");
  if (a->num_pages < 1) return fail(KVSKIP_E_INVALID, "paged cache: num_pages >= 1");
  if (a->bt_stride < nb) return fail(KVSKIP_E_INVALID, "paged cache: block_table rows must hold ceil(T / 64) pages");
  const int64_t per = a->seq_lens != nullptr ? (a->B * items + a->num_splits - 1) / a->num_splits
                                             : (items + a->num_splits - 1) / a->num_splits;
  if (per > kvs::planner_max_blocks(1))
    return fail(KVSKIP_E_UNSUPPORTED, "paged cache: at most %d blocks per split (raise num_splits)",
                kvs::planner_max_blocks(1));
  return KVSKIP_OK;
}

static int check_decode(const kvskip_attn_args* a, int stats, int load_v, int phase, kvs::AttnP* p) {
  int rc = prepare_attn(a, true, true, load_v != 0, p);
  if (rc != KVSKIP_OK) return rc;
  if (!load_v && !stats) return fail(KVSKIP_E_INVALID, "load_v=false only makes sense with stats=true");
  if (a->p_out != nullptr && !stats) return fail(KVSKIP_E_INVALID, "write_p needs stats=true");
  if (load_v && a->out == nullptr) return fail(KVSKIP_E_INVALID, "out is required with load_v");
  if (stats && (a->blk_max == nullptr || a->blk_sum == nullptr))
    return fail(KVSKIP_E_INVALID, "stats needs blk_max and blk_sum");
  if (load_v && a->num_splits > 1 && a->part_acc == nullptr)
    return fail(KVSKIP_E_INVALID, "num_splits > 1 needs the split partial buffers");
  const bool masked = a->block_idx != nullptr;
  if (masked) {
    if (a->block_cnt == nullptr) return fail(KVSKIP_E_INVALID, "block_cnt is required with block_idx");
    if (a->max_blocks < 0) return fail(KVSKIP_E_INVALID, "block_idx must be contiguous int32 [B, Hkv, max_blocks]");
  }
  if (phase != 3 && a->num_splits < 2) return fail(KVSKIP_E_INVALID, "decode phases need num_splits >= 2");
  if (a->seq_lens != nullptr) {
    if (a->num_splits < 2) return fail(KVSKIP_E_INVALID, "seq_lens needs num_splits >= 2");
    if (a->B > kvs::MAX_RAGGED_B) return fail(KVSKIP_E_UNSUPPORTED, "seq_lens: B <= %d", kvs::MAX_RAGGED_B);
    if (a->p_out != nullptr) return fail(KVSKIP_E_UNSUPPORTED, "seq_lens: no fp16 P output");
  }
  if (a->list_partition != 0) {
    if (a->list_partition != 1) return fail(KVSKIP_E_INVALID, "list_partition in {0, 1}");
    if (!masked || a->seq_lens == nullptr)
      return fail(KVSKIP_E_INVALID, "list_partition 1 partitions a masked ragged pass (block_idx and seq_lens)");
    if (a->B * a->Hkv > kvs::MAX_GLOBAL_LISTS)
      return fail(KVSKIP_E_UNSUPPORTED, "list_partition 1: B * Hkv <= %d", kvs::MAX_GLOBAL_LISTS);
  }
  if (a->block_table != nullptr && (phase & 1)) {  // paged cache (the merge alone reads no K / V)
    const int rc = check_paged(a, p->nb, masked ? a->max_blocks : p->nb);
    if (rc != KVSKIP_OK) return rc;
  }
  if (!load_v) p->out = nullptr;
  return KVSKIP_OK;
}

static int decode_phases(const kvskip_attn_args* a, int stats, int load_v, int phase, void* stream) {
  kvs::AttnP p;
  const int rc = check_decode(a, stats, load_v, phase, &p);
  if (rc != KVSKIP_OK) return rc;
  const int G = a->Hq / a->Hkv;
  return launched(kvs::launch_decode(p, a->D, G, a->block_idx != nullptr, stats != 0, load_v != 0, phase,
                                     static_cast<hipStream_t>(stream)),
                  "kvskip_decode");
}

int kvskip_decode(const kvskip_attn_args* a, int stats, int load_v, void* stream) {
  return decode_phases(a, stats, load_v, 3, stream);
}

int kvskip_decode_splits(const kvskip_attn_args* a, int stats, int load_v, void* stream) {
  return decode_phases(a, stats, load_v, 1, stream);
}

int kvskip_merge_splits(const kvskip_attn_args* a, int stats, int load_v, void* stream) {
  return decode_phases(a, stats, load_v, 2, stream);
}

int kvskip_decode_scratch(const kvskip_attn_args* a, int stats, int load_v, void* stream) {
  if (a == nullptr) return fail(KVSKIP_E_INVALID, "null argument block");
  // The partials live in `scratch`: part_acc [B, Hq, S, D] (with V) then part_ml [B, Hq, S, 2],
  // each 256-byte aligned. Sizes are checked before any device call.
  const int64_t S = a->num_splits;
  int64_t acc_floats = 0, need = 0;
  if (S > 1 && a->B > 0 && a->Hq > 0 && a->D > 0) {
    const int64_t rows = static_cast<int64_t>(a->B) * a->Hq * S;
    acc_floats = load_v ? (rows * a->D + 63) / 64 * 64 : 0;
    need = acc_floats + rows * 2;
    if (need > SCRATCH_FLOATS)
      return fail(KVSKIP_E_INVALID,
                  "kvskip_decode_scratch: split partials need %lld bytes, the scratch holds %lld "
                  "(B * Hq * num_splits * (D + 2) * 4 bytes at most; lower num_splits or call kvskip_decode)",
                  static_cast<long long>(need * 4), static_cast<long long>(KVSKIP_SCRATCH_BYTES));
  }
  kvskip_attn_args as = *a;
  as.part_acc = nullptr;
  as.part_ml = nullptr;
  if (S > 1) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(KVSKIP_E_LAUNCH, "kvskip_decode_scratch: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= SCRATCH_MAX_DEVICES)
      return fail(KVSKIP_E_UNSUPPORTED, "kvskip_decode_scratch: device %d beyond %d", dev, SCRATCH_MAX_DEVICES);
    float* base;
    {
      // first call on this device (current here): the device's own address of the array
      std::lock_guard<std::mutex> lk(g_scratch_mu);
      if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || ptr == nullptr)
          return fail(KVSKIP_E_LAUNCH, "kvskip_decode_scratch: hipGetSymbolAddress: %s", hipGetErrorString(e));
        g_scratch_ptr[dev] = static_cast<float*>(ptr);
      }
      base = g_scratch_ptr[dev];
    }
    as.part_acc = load_v ? base : nullptr;
    as.part_ml = base + acc_floats;
  }
  return decode_phases(&as, stats, load_v, 3, stream);
}

int kvskip_pv(const kvskip_attn_args* a, void* stream) {
  kvs::AttnP p;
  int rc = prepare_attn(a, false, false, true, &p);
  if (rc != KVSKIP_OK) return rc;
  if (a->seq_lens != nullptr) return fail(KVSKIP_E_UNSUPPORTED, "pv: seq_lens is not supported");
  if (a->block_table != nullptr) {
    rc = check_paged(a, p.nb, a->max_blocks);
    if (rc != KVSKIP_OK) return rc;
  }
  if (a->p_in == nullptr) return fail(KVSKIP_E_INVALID, "P: fp16 [B, Hq, t_pad]");
  if (!aligned16(a->p_in)) return fail(KVSKIP_E_INVALID, "P must be 16-byte aligned");
  if (a->blk_scale == nullptr) return fail(KVSKIP_E_INVALID, "blk_scale: contiguous fp32 [B, Hkv, nb, G]");
  if (a->block_idx == nullptr) return fail(KVSKIP_E_INVALID, "block_idx");
  if (a->block_cnt == nullptr) return fail(KVSKIP_E_INVALID, "block_cnt");
  if (a->out == nullptr) return fail(KVSKIP_E_INVALID, "out is required");
  if (a->num_splits > 1 && a->part_acc == nullptr)
    return fail(KVSKIP_E_INVALID, "num_splits > 1 needs the split partial buffers");
  const int G = a->Hq / a->Hkv;
  return launched(kvs::launch_pv(p, a->D, G, static_cast<hipStream_t>(stream)), "kvskip_pv");
}

int kvskip_vskip1(const kvskip_attn_args* a, void* stream) {
  kvs::AttnP p;
  int rc = prepare_attn(a, true, true, true, &p);
  if (rc != KVSKIP_OK) return rc;
  if (a->seq_lens != nullptr) return fail(KVSKIP_E_UNSUPPORTED, "vskip1: seq_lens is not supported");
  if (a->block_table != nullptr) {
    rc = check_paged(a, p.nb, p.nb);
    if (rc != KVSKIP_OK) return rc;
  }
  if (!(a->tau > 0.f) || a->local < 0) return fail(KVSKIP_E_INVALID, "tau > 0, local >= 0, num_splits >= 1");
  if (a->out == nullptr) return fail(KVSKIP_E_INVALID, "out is required");
  if (a->num_splits > 1 && a->part_acc == nullptr)
    return fail(KVSKIP_E_INVALID, "num_splits > 1 needs the split partial buffers");
  p.log2_tau = static_cast<float>(std::log2(static_cast<double>(a->tau)));
  const int G = a->Hq / a->Hkv;
  return launched(kvs::launch_vskip1(p, a->D, G, static_cast<hipStream_t>(stream)), "kvskip_vskip1");
}

int kvskip_read(const void* x, int64_t bytes, uint32_t* out, int32_t blocks, void* stream) {
  if (x == nullptr || out == nullptr) return fail(KVSKIP_E_INVALID, "x: contiguous CUDA, 16-byte multiple");
  if (bytes % 16 != 0 || !aligned16(x)) return fail(KVSKIP_E_INVALID, "x: contiguous CUDA, 16-byte multiple");
  if (blocks < 1) return fail(KVSKIP_E_INVALID, "blocks >= 1");
  return launched(kvs::launch_read(x, bytes, out, blocks, static_cast<hipStream_t>(stream)), "kvskip_read");
}

static int check_plan(const kvskip_plan_args* p) {
  if (p == nullptr) return fail(KVSKIP_E_INVALID, "null argument block");
  if (p->q == nullptr || p->k == nullptr) return fail(KVSKIP_E_INVALID, "q: CUDA bf16 [B, Hq, D]");
  if (p->B < 1 || p->Hkv < 1 || p->Hq < 1 || p->T < 1) return fail(KVSKIP_E_INVALID, "sizes must be positive");
  if (p->Hq % p->Hkv != 0) return fail(KVSKIP_E_INVALID, "Hq must be a multiple of Hkv");
  const int G = p->Hq / p->Hkv;
  if (!((p->D == 64 || p->D == 128) && (G == 1 || G == 2 || G == 4 || G == 7 || G == 8)))
    return fail(KVSKIP_E_UNSUPPORTED, "planner kernels: D in {64, 128}, G in {1, 2, 4, 7, 8} (D=%d, G=%d)", p->D, G);
  int rc = check_kv(p->k, p->k_sb, p->k_sh, p->k_st, "k");
  if (rc != KVSKIP_OK) return rc;
  if (p->csum == nullptr || p->lse_ref == nullptr || p->cs_ref == nullptr || p->keep == nullptr ||
      p->lse_att == nullptr || p->age == nullptr || p->flags == nullptr || p->cs_now == nullptr ||
      p->trig == nullptr || p->block_idx == nullptr || p->block_cnt == nullptr)
    return fail(KVSKIP_E_INVALID, "plan: missing state tensor");
  if (!aligned16(p->csum)) return fail(KVSKIP_E_INVALID, "csum must be 16-byte aligned");
  const int nb = (p->T + KVSKIP_BLOCK - 1) / KVSKIP_BLOCK;
  if (nb > p->NBC) return fail(KVSKIP_E_INVALID, "block capacity exceeded");
  if (nb > kvs::planner_max_blocks(G))
    return fail(KVSKIP_E_UNSUPPORTED, "plan: %d blocks exceed the planner capacity (%d)", nb, kvs::planner_max_blocks(G));
  if (p->ids != nullptr) {
    if (p->part == nullptr || p->idx_out == nullptr || p->idx != nullptr)
      return fail(KVSKIP_E_INVALID, "plan: ids needs part and idx_out, and no idx");
    if (p->ids_sb < p->T) return fail(KVSKIP_E_INVALID, "plan: ids rows must hold >= T tokens");
  }
  if (p->aix != nullptr && p->idx == nullptr && p->ids == nullptr) return fail(KVSKIP_E_INVALID, "aix needs idx");
  if (p->calib_kind < 0 || p->calib_kind > 2) return fail(KVSKIP_E_INVALID, "calib_kind in {0, 1, 2}");
  if (p->block_table != nullptr && (p->num_pages < 1 || p->bt_stride < nb))
    return fail(KVSKIP_E_INVALID, "paged cache: num_pages >= 1 and block_table rows of ceil(T / 64) pages");
  return KVSKIP_OK;
}

int kvskip_plan(const kvskip_plan_args* p, void* stream) {
  const int rc = check_plan(p);
  if (rc != KVSKIP_OK) return rc;
  if (p->ticket != nullptr && p->part == nullptr) return fail(KVSKIP_E_INVALID, "plan: ticket needs the part workspace");
  return launched(kvs::launch_plan(*p, static_cast<hipStream_t>(stream)), "kvskip_plan");
}

int kvskip_plan_scores(const kvskip_plan_args* p, void* stream) {
  const int rc = check_plan(p);
  if (rc != KVSKIP_OK) return rc;
  if (p->part == nullptr) return fail(KVSKIP_E_INVALID, "plan_scores needs the part workspace");
  return launched(kvs::launch_plan_scores(*p, static_cast<hipStream_t>(stream)), "kvskip_plan_scores");
}

int64_t kvskip_plan_part_floats(int32_t B, int32_t Hq, int32_t Hkv, int32_t NBC) {
  if (B < 1 || Hkv < 1 || Hq < 1 || NBC < 1 || Hq % Hkv != 0) return -1;
  return kvs::plan_part_floats(B, Hq, Hkv, NBC);
}

static int check_update(const kvskip_update_args* p) {
  if (p == nullptr) return fail(KVSKIP_E_INVALID, "null argument block");
  if (p->blk_max == nullptr || p->blk_sum == nullptr) return fail(KVSKIP_E_INVALID, "blk_max must be contiguous CUDA fp32");
  if (p->trig == nullptr || p->cs_now == nullptr || p->keep == nullptr || p->lse_ref == nullptr ||
      p->cs_ref == nullptr || p->lse_att == nullptr)
    return fail(KVSKIP_E_INVALID, "update: missing state tensor");
  if (p->B < 1 || p->Hkv < 1 || p->Hq < 1 || p->T < 1) return fail(KVSKIP_E_INVALID, "sizes must be positive");
  if (p->Hq % p->Hkv != 0) return fail(KVSKIP_E_INVALID, "Hq must be a multiple of Hkv");
  const int G = p->Hq / p->Hkv;
  if (!(G == 1 || G == 2 || G == 4 || G == 7 || G == 8))
    return fail(KVSKIP_E_UNSUPPORTED, "planner kernels: G in {1, 2, 4, 7, 8} (G=%d)", G);
  const int nb = (p->T + KVSKIP_BLOCK - 1) / KVSKIP_BLOCK;
  if (nb > p->NBC) return fail(KVSKIP_E_INVALID, "block capacity exceeded");
  if (nb > kvs::planner_max_blocks(G))
    return fail(KVSKIP_E_UNSUPPORTED, "update: %d blocks exceed the planner capacity (%d)", nb, kvs::planner_max_blocks(G));
  if (p->calib != nullptr) {
    if (p->flags == nullptr || p->est == nullptr) return fail(KVSKIP_E_INVALID, "calibration needs flags and est");
    if (p->calib_kind < 0 || p->calib_kind > 2) return fail(KVSKIP_E_INVALID, "calib_kind in {0, 1, 2}");
  }
  if (p->aix != nullptr && p->idx == nullptr) return fail(KVSKIP_E_INVALID, "aix needs idx");
  if (p->list_stats && p->flags == nullptr) return fail(KVSKIP_E_INVALID, "list_stats needs flags");
  return KVSKIP_OK;
}

int kvskip_update(const kvskip_update_args* p, void* stream) {
  const int rc = check_update(p);
  if (rc != KVSKIP_OK) return rc;
  return launched(kvs::launch_update(*p, static_cast<hipStream_t>(stream)), "kvskip_update");
}

int kvskip_merge_update(const kvskip_attn_args* a, const kvskip_update_args* u, void* stream) {
  kvs::AttnP p;
  int rc = prepare_attn(a, false, false, false, &p);
  if (rc != KVSKIP_OK) return rc;
  if ((rc = check_update(u)) != KVSKIP_OK) return rc;
  if (a->num_splits < 2 || a->part_acc == nullptr) return fail(KVSKIP_E_INVALID, "merge_update needs num_splits >= 2");
  if (a->out == nullptr) return fail(KVSKIP_E_INVALID, "out is required with load_v");
  if (a->B != u->B || a->Hq != u->Hq || a->Hkv != u->Hkv || a->T != u->T)
    return fail(KVSKIP_E_INVALID, "merge_update: attention and update shapes differ");
  return launched(kvs::launch_merge_update(p, *u, a->D, static_cast<hipStream_t>(stream)), "kvskip_merge_update");
}

int kvskip_decode_splits_update(const kvskip_attn_args* a, const kvskip_update_args* u, void* stream) {
  kvs::AttnP p;
  int rc = check_decode(a, 1, 1, a != nullptr && a->num_splits > 1 ? 1 : 3, &p);
  if (rc != KVSKIP_OK) return rc;
  if ((rc = check_update(u)) != KVSKIP_OK) return rc;
  if (a->block_idx == nullptr) return fail(KVSKIP_E_INVALID, "decode_splits_update: the pass needs a block list");
  if (a->Hq / a->Hkv != u->Hq / u->Hkv)
    return fail(KVSKIP_E_INVALID, "decode_splits_update: the pass and the update have different group sizes");
  return launched(kvs::launch_split_update(p, *u, a->D, static_cast<hipStream_t>(stream)), "kvskip_decode_splits_update");
}

int kvskip_decode_splits_planned(const kvskip_attn_args* a, const kvskip_plan_args* pl, const kvskip_update_args* u,
                                 void* stream) {
  int rc = check_plan(pl);
  if (rc != KVSKIP_OK) return rc;
  if (a == nullptr) return fail(KVSKIP_E_INVALID, "null argument block");
  if (pl->part == nullptr) return fail(KVSKIP_E_INVALID, "decode_splits_planned needs the plan's part workspace");
  if (pl->seq_lens != a->seq_lens)
    return fail(KVSKIP_E_INVALID, "decode_splits_planned: the plan and the pass must share seq_lens");
  if (a->seq_lens != nullptr && a->B > 1) {  // a ragged batch: the ragged partition over the decided lists
    if (a->B > 16)
      return fail(KVSKIP_E_UNSUPPORTED, "decode_splits_planned: a ragged batch of at most 16 sequences (got %d; plan "
                                        "and decide separately for more)", a->B);
    if (a->block_table != nullptr)
      return fail(KVSKIP_E_UNSUPPORTED, "decode_splits_planned: a ragged batch reads a contiguous cache");
    if (a->list_partition != 0)
      return fail(KVSKIP_E_UNSUPPORTED, "decode_splits_planned: a ragged batch's lists are decided per KV head "
                                        "(list_partition 0)");
    if (pl->pass_budget != 0 || pl->slot_base != 0 || pl->slot_count != 0 || pl->lse_part != nullptr ||
        pl->decide_mode == KVSKIP_DECIDE_POST)
      return fail(KVSKIP_E_UNSUPPORTED, "decode_splits_planned: a ragged batch takes no pass_budget, slots, lse_part "
                                        "or DECIDE_POST");
  }
  if (a->B != pl->B || a->Hq != pl->Hq || a->Hkv != pl->Hkv || a->T != pl->T || a->D != pl->D)
    return fail(KVSKIP_E_INVALID, "decode_splits_planned: attention and plan shapes differ");
  if (pl->decide_mode < KVSKIP_DECIDE_PLAN || pl->decide_mode > KVSKIP_DECIDE_POST)
    return fail(KVSKIP_E_INVALID, "decode_splits_planned: decide_mode in {0, 1, 2} (got %d)", pl->decide_mode);
  if (pl->slot_base < 0 || pl->slot_count < 0 ||
      (pl->slot_count > 0 ? pl->slot_base + pl->slot_count : pl->slot_base + a->num_splits) > a->num_splits)
    return fail(KVSKIP_E_INVALID, "decode_splits_planned: slots [slot_base, slot_base + slot_count) within num_splits");
  if (pl->lse_part != nullptr &&
      (pl->lse_slots < 1 || pl->lse_slots > 64 || pl->lse_stride < pl->lse_slots))
    return fail(KVSKIP_E_INVALID, "decode_splits_planned: lse_slots in 1..64, lse_stride >= lse_slots");
  if (pl->pass_budget < 0 || pl->pass_budget > 65536)
    return fail(KVSKIP_E_INVALID, "decode_splits_planned: pass_budget in 0..65536");
  if (pl->pass_budget > 0 && a->B * a->Hkv > 16)
    return fail(KVSKIP_E_UNSUPPORTED, "decode_splits_planned: pass_budget needs B * Hkv <= 16 (got %d)", a->B * a->Hkv);
  kvskip_attn_args am = *a;  // the pass's list is the plan's
  am.block_idx = pl->block_idx;
  am.block_cnt = pl->block_cnt;
  am.max_blocks = pl->NBC;
  kvs::AttnP p;
  if ((rc = check_decode(&am, 1, 1, a->num_splits > 1 ? 1 : 3, &p)) != KVSKIP_OK) return rc;
  if (u != nullptr && (rc = check_update(u)) != KVSKIP_OK) return rc;
  return launched(kvs::launch_planned_split(p, *pl, u, a->D, static_cast<hipStream_t>(stream)),
                  "kvskip_decode_splits_planned");
}

static int check_select(const kvskip_select_args* s) {
  if (s == nullptr) return fail(KVSKIP_E_INVALID, "null argument block");
  if (s->blk_max == nullptr || s->blk_sum == nullptr) return fail(KVSKIP_E_INVALID, "select: blk_max / blk_sum");
  if (s->B < 1 || s->Hq < 1 || s->Hkv < 1 || s->nb < 1) return fail(KVSKIP_E_INVALID, "sizes must be positive");
  if (s->Hq % s->Hkv != 0) return fail(KVSKIP_E_INVALID, "Hq must be a multiple of Hkv");
  if (s->Hq / s->Hkv > 8) return fail(KVSKIP_E_UNSUPPORTED, "select: G <= 8 (G=%d)", s->Hq / s->Hkv);
  if (s->nb > kvs::planner_max_blocks(1))
    return fail(KVSKIP_E_UNSUPPORTED, "select: at most %d blocks (nb=%d)", kvs::planner_max_blocks(1), s->nb);
  if (s->rule != 0 && s->rule != 1) return fail(KVSKIP_E_INVALID, "rule must be tau or topp");
  if (!(s->value > 0.f) || s->local < 0) return fail(KVSKIP_E_INVALID, "select: value > 0, local >= 0");
  if (s->block_idx != nullptr && s->block_cnt == nullptr) return fail(KVSKIP_E_INVALID, "block_cnt is required with block_idx");
  return KVSKIP_OK;
}

int kvskip_select(const kvskip_select_args* s, void* stream) {
  const int rc = check_select(s);
  if (rc != KVSKIP_OK) return rc;
  return launched(kvs::launch_select(*s, static_cast<hipStream_t>(stream)), "kvskip_select");
}

int kvskip_pv_select(const kvskip_attn_args* a, const kvskip_select_args* s, void* stream) {
  int rc = check_select(s);
  if (rc != KVSKIP_OK) return rc;
  kvs::AttnP p;
  if ((rc = prepare_attn(a, false, false, true, &p)) != KVSKIP_OK) return rc;
  if (a->seq_lens != nullptr || a->block_table != nullptr)
    return fail(KVSKIP_E_UNSUPPORTED, "pv_select: a contiguous cache without seq_lens (else kvskip_select, kvskip_pv)");
  if (s->B != a->B || s->Hq != a->Hq || s->Hkv != a->Hkv || s->nb != p.nb)
    return fail(KVSKIP_E_INVALID, "pv_select: the selection's B, Hq, Hkv, nb differ from the pass's");
  if (a->p_in == nullptr) return fail(KVSKIP_E_INVALID, "P: fp16 [B, Hq, t_pad]");
  if (!aligned16(a->p_in)) return fail(KVSKIP_E_INVALID, "P must be 16-byte aligned");
  if (a->out == nullptr) return fail(KVSKIP_E_INVALID, "out is required");
  if (a->num_splits > 1 && a->part_acc == nullptr)
    return fail(KVSKIP_E_INVALID, "num_splits > 1 needs the split partial buffers");
  return launched(kvs::launch_pv_select(p, *s, a->D, a->Hq / a->Hkv, static_cast<hipStream_t>(stream)),
                  "kvskip_pv_select");
}

int kvskip_block_list(const uint8_t* keep, int32_t B, int32_t Hkv, int32_t nb, int32_t* block_idx,
                      int32_t* block_cnt, void* stream) {
  if (keep == nullptr || block_idx == nullptr || block_cnt == nullptr)
    return fail(KVSKIP_E_INVALID, "block_list: null tensor");
  if (B < 1 || Hkv < 1 || nb < 1) return fail(KVSKIP_E_INVALID, "sizes must be positive");
  return launched(kvs::launch_block_list(keep, B, Hkv, nb, block_idx, block_cnt, static_cast<hipStream_t>(stream)),
                  "kvskip_block_list");
}

int kvskip_block_sums(const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st, int32_t B, int32_t Hkv, int32_t T,
                      int32_t D, float* csum, int32_t NBC, const int32_t* seq_lens, const int32_t* block_table,
                      int64_t bt_stride, int32_t num_pages, void* stream) {
  if (k == nullptr || csum == nullptr) return fail(KVSKIP_E_INVALID, "block_sums: null tensor");
  if (B < 1 || Hkv < 1 || T < 1) return fail(KVSKIP_E_INVALID, "sizes must be positive");
  if (D != 64 && D != 128) return fail(KVSKIP_E_UNSUPPORTED, "block_sums: D in {64, 128}");
  if ((T + KVSKIP_BLOCK - 1) / KVSKIP_BLOCK > NBC) return fail(KVSKIP_E_INVALID, "block capacity exceeded");
  if (k_st % 8 != 0 || k_sh % 8 != 0 || k_sb % 8 != 0 || !aligned16(k))
    return fail(KVSKIP_E_INVALID, "k strides must be multiples of 8 elements (16-byte rows)");
  if (block_table != nullptr && (num_pages < 1 || bt_stride < (T + KVSKIP_BLOCK - 1) / KVSKIP_BLOCK))
    return fail(KVSKIP_E_INVALID, "paged cache: num_pages >= 1 and block_table rows of ceil(T / 64) pages");
  return launched(kvs::launch_block_sums(k, k_sb, k_sh, k_st, B, Hkv, T, D, csum, NBC, seq_lens, block_table,
                                         bt_stride, num_pages, static_cast<hipStream_t>(stream)),
                  "kvskip_block_sums");
}

int kvskip_token_index(const int32_t* ids, int64_t ids_stride, int32_t B, int32_t T, uint8_t* idx, int32_t NBC,
                       const int32_t* seq_lens, void* stream) {
  if (ids == nullptr || idx == nullptr) return fail(KVSKIP_E_INVALID, "token_index: null tensor");
  if (B < 1 || T < 1 || ids_stride < T) return fail(KVSKIP_E_INVALID, "token_index: ids must be [B, >= T] int32");
  if ((T + KVSKIP_BLOCK - 1) / KVSKIP_BLOCK > NBC) return fail(KVSKIP_E_INVALID, "block capacity exceeded");
  return launched(kvs::launch_token_index(ids, ids_stride, B, T, idx, NBC, seq_lens, static_cast<hipStream_t>(stream)),
                  "kvskip_token_index");
}

}  // extern "C"
