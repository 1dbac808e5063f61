// Device helpers shared by the kvskip_amd kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kvskip_amd.h"

namespace kvs {

constexpr int BLK = KVSKIP_BLOCK;            // tokens per block (mask / stats granularity)
constexpr int WAVE = 64;
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
constexpr float NEG_INF = -__builtin_huge_valf();

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// bf16 pair packed in a dword -> the two fp32 values (exact).
__device__ __forceinline__ float bf_lo(uint32_t x) { return __uint_as_float(x << 16); }
__device__ __forceinline__ float bf_hi(uint32_t x) { return __uint_as_float(x & 0xffff0000u); }

// fp32 -> bf16 bits, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// fp16 bits <-> fp32 (hardware conversions).
__device__ __forceinline__ float h2f(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f)); }

// a.x*b.x + a.y*b.y + c over packed bf16 pairs, fp32 accumulate (v_dot2_f32_bf16).
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                         false);
}
__device__ __forceinline__ float dot8(const u32x4& a, const u32x4& b, float c) {
  c = dot2(a.x, b.x, c);
  c = dot2(a.y, b.y, c);
  c = dot2(a.z, b.z, c);
  return dot2(a.w, b.w, c);
}

__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }  // v_exp_f32
__device__ __forceinline__ float flog2(float x) { return __builtin_amdgcn_logf(x); }   // v_log_f32

// DPP lane permutations (row = 16 lanes).
enum : int {
  DPP_XOR1 = 0xB1,         // quad_perm [1,0,3,2]
  DPP_XOR2 = 0x4E,         // quad_perm [2,3,0,1]
  DPP_HALF_MIRROR = 0x141, // lane i <-> 7 - i within each 8
  DPP_MIRROR = 0x140,      // lane i <-> 15 - i within each 16
  DPP_ROR8 = 0x128         // lane i <-> i ^ 8 within each 16
};

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_amdgcn_update_dpp(0.f, v, CTRL, 0xF, 0xF, false);
}

// Sum over the 8 lanes of each aligned group of 8 (every lane gets the group sum).
__device__ __forceinline__ float sum8(float v) {
  v += dpp<DPP_XOR1>(v);
  v += dpp<DPP_XOR2>(v);
  v += dpp<DPP_HALF_MIRROR>(v);
  return v;
}

__device__ __forceinline__ float xshfl(float v, int mask) { return __shfl_xor(v, mask, WAVE); }

// Value of lane `src` as a wavefront-uniform (scalar) value.
__device__ __forceinline__ float lane_value(float v, int src) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}

// Combine the four 16-lane rows of a row-reduced value (uniform result, fixed order).
__device__ __forceinline__ float rows4_sum(float v) {
  return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}
__device__ __forceinline__ float rows4_max(float v) {
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

// Reductions over lane bits 3..5 (the 8 row slots of the K layout; values are equal within each
// aligned group of 8 lanes); the result is wavefront-uniform.
__device__ __forceinline__ float max_rows8(float v) { return rows4_max(fmaxf(v, dpp<DPP_ROR8>(v))); }
__device__ __forceinline__ float sum_rows8(float v) { return rows4_sum(v + dpp<DPP_ROR8>(v)); }

// Whole-wavefront reductions (uniform result): DPP inside the 16-lane rows, then the 4 rows.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<DPP_XOR1>(v);
  v += dpp<DPP_XOR2>(v);
  v += dpp<DPP_HALF_MIRROR>(v);
  v += dpp<DPP_MIRROR>(v);
  return rows4_sum(v);
}
// Integer wavefront scan (inclusive, over lanes) and sum; uniform sum. DPP shifts inside each
// 16-lane row (0 from outside the row), then the totals of the rows before.
template <int CTRL>
__device__ __forceinline__ int dpp_i0(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}
__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = threadIdx.x % WAVE;
  v += dpp_i0<0x111>(v);  // row_shr:1
  v += dpp_i0<0x112>(v);  // row_shr:2
  v += dpp_i0<0x114>(v);  // row_shr:4
  v += dpp_i0<0x118>(v);  // row_shr:8
  const int t0 = __builtin_amdgcn_readlane(v, 15), t1 = __builtin_amdgcn_readlane(v, 31),
            t2 = __builtin_amdgcn_readlane(v, 47);
  const int row = lane >> 4;
  return v + (row == 0 ? 0 : row == 1 ? t0 : row == 2 ? t0 + t1 : t0 + t1 + t2);
}
__device__ __forceinline__ int wave_sum_int(int v) {
  return __builtin_amdgcn_readlane(wave_incl_scan(v), WAVE - 1);
}

// Unsigned integer minimum over the wavefront (uniform result).
template <int CTRL>
__device__ __forceinline__ uint32_t dppu(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ uint32_t lane_u32(uint32_t v, int src) {
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), src));
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  v = min(v, dppu<DPP_XOR1>(v));
  v = min(v, dppu<DPP_XOR2>(v));
  v = min(v, dppu<DPP_HALF_MIRROR>(v));
  v = min(v, dppu<DPP_MIRROR>(v));
  return min(min(lane_u32(v, 0), lane_u32(v, 16)), min(lane_u32(v, 32), lane_u32(v, 48)));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<DPP_XOR1>(v));
  v = fmaxf(v, dpp<DPP_XOR2>(v));
  v = fmaxf(v, dpp<DPP_HALF_MIRROR>(v));
  v = fmaxf(v, dpp<DPP_MIRROR>(v));
  return rows4_max(v);
}

// 16-byte loads: plain and streaming (non-temporal).
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ u32x4 ld16_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Raw buffer access: an SGPR resource over [base, base + bytes), 32-bit lane offsets and a
// uniform SGPR offset; loads past the range return zeros.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}
constexpr int BUF_NT = 2;  // cache policy: non-temporal
template <int AUX = 0>
__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff), static_cast<int>(soff), AUX);
}

// 4- and 2-byte stores through a buffer resource: per-lane 32-bit offset + scalar offset, so a
// loop keeps one offset register per store stream instead of a 64-bit address.
__device__ __forceinline__ void bstore_f32(float v, rsrc_t r, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, static_cast<int>(voff), static_cast<int>(soff), 0);
}
__device__ __forceinline__ void bstore_u16(uint16_t v, rsrc_t r, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b16(v, r, static_cast<int>(voff), static_cast<int>(soff), 0);
}

// Online log-sum-exp accumulator in natural units (planner): (m, s) with s = sum exp(x - m).
__device__ __forceinline__ void lse_push(float& m, float& s, float x) {
  if (x == NEG_INF) return;
  if (x > m) {
    s = s * __expf(m - x) + 1.f;
    m = x;
  } else {
    s += __expf(x - m);
  }
}

}  // namespace kvs
