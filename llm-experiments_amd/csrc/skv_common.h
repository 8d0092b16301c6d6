// Shared device helpers for the simple-kv (skv) HIP kernels on gfx950 (CDNA4).
//
// Storage types: fp32 (`float`) and bf16 (raw `uint16_t`, round-to-nearest-even
// on store). All arithmetic is fp32. Cross-lane reductions use DPP row
// operations, which stay inside one 16-lane row of a 64-lane wavefront.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "skv.h"

namespace skv {

// ---------------------------------------------------------------------------
// bf16 <-> fp32
// ---------------------------------------------------------------------------

// fp32 -> bf16 with round-to-nearest-even; NaN maps to a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}

// A 32-bit word holding two bf16 values: element 0 in bits 0..15, element 1
// in bits 16..31 (little-endian memory order).
__device__ __forceinline__ float bf16w_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16w_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// ---------------------------------------------------------------------------
// Per-lane fragments of one K/V row.
//
// A token row of D elements is split over the 16 lanes of a DPP row: lane i
// owns elements [i*EPL, (i+1)*EPL), EPL = D/16. Frag<TC, EPL> keeps the raw
// words (so bf16 rows stay packed in registers until use) and converts one
// element at a time.
// ---------------------------------------------------------------------------

template <typename TC, int EPL>
struct Frag;

// K/V rows are read exactly once per call, so every fragment load is
// non-temporal (the nt bit on global_load): streaming a 1 GB cache this way
// measured ~13% faster on MI355X than ordinary loads.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ u32x4_t stream_load16(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
}
__device__ __forceinline__ u32x2_t stream_load8(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
}

template <int EPL>
struct Frag<float, EPL> {
  static constexpr int NW = EPL;  // 32-bit words
  uint32_t w[NW];
  __device__ __forceinline__ void load(const float* p) {
    static_assert(EPL % 4 == 0, "fp32 fragment must be a multiple of 16 bytes");
#pragma unroll
    for (int i = 0; i < NW / 4; ++i) {
      const u32x4_t x = stream_load16(p + 4 * i);
      w[4 * i + 0] = x.x; w[4 * i + 1] = x.y; w[4 * i + 2] = x.z; w[4 * i + 3] = x.w;
    }
  }
  __device__ __forceinline__ float get(int e) const { return __uint_as_float(w[e]); }
};

template <int EPL>
struct Frag<uint16_t, EPL> {
  static constexpr int NW = EPL / 2;
  uint32_t w[NW];
  __device__ __forceinline__ void load(const uint16_t* p) {
    if constexpr (NW % 4 == 0) {
#pragma unroll
      for (int i = 0; i < NW / 4; ++i) {
        const u32x4_t x = stream_load16(p + 8 * i);
        w[4 * i + 0] = x.x; w[4 * i + 1] = x.y; w[4 * i + 2] = x.z; w[4 * i + 3] = x.w;
      }
    } else {
      static_assert(NW == 2, "bf16 fragment must be 8 or a multiple of 16 bytes");
      const u32x2_t x = stream_load8(p);
      w[0] = x.x; w[1] = x.y;
    }
  }
  __device__ __forceinline__ float get(int e) const {
    return (e & 1) ? bf16w_hi(w[e >> 1]) : bf16w_lo(w[e >> 1]);
  }
};

// Eight consecutive elements of a runtime-dtype row, as fp32, with one branch
// and vector loads (p + i must be 16-byte aligned for fp32, 8 elements
// aligned for bf16). A per-element load behind a dtype branch makes the
// compiler wait for each load on its own.
__device__ __forceinline__ void load8_f32(const void* p, size_t i, int dt, float* out) {
  if (dt == SKV_BF16) {
    const uint4 x = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i);
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      out[2 * j] = bf16w_lo(w[j]);
      out[2 * j + 1] = bf16w_hi(w[j]);
    }
  } else {
    const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
    const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i + 4);
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  }
}

// Four consecutive elements, as load8_f32 (p + i 16-byte aligned for fp32,
// 8-byte aligned for bf16).
__device__ __forceinline__ void load4_f32(const void* p, size_t i, int dt, float* out) {
  if (dt == SKV_BF16) {
    const uint2 x = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i);
    out[0] = bf16w_lo(x.x);
    out[1] = bf16w_hi(x.x);
    out[2] = bf16w_lo(x.y);
    out[3] = bf16w_hi(x.y);
  } else {
    const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
  }
}

// Element loads/stores with runtime dtype (used off the hot loops).
__device__ __forceinline__ float load_elem(const void* p, size_t i, int dt) {
  return dt == SKV_BF16 ? bf16_to_f32(static_cast<const uint16_t*>(p)[i])
                        : static_cast<const float*>(p)[i];
}
__device__ __forceinline__ void store_elem(void* p, size_t i, int dt, float v) {
  if (dt == SKV_BF16) static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
  else static_cast<float*>(p)[i] = v;
}

// ---------------------------------------------------------------------------
// DPP reductions over one 16-lane row. Every lane of the row ends with the
// same bit pattern: each step combines a lane with a partner that holds the
// mirror-image partial, and fp add/max are commutative.
//   quad_perm [1,0,3,2]  partner = lane ^ 1
//   quad_perm [2,3,0,1]  partner = lane ^ 2
//   row_half_mirror      partner = 7 - lane (within each half-row)
//   row_mirror           partner = 15 - lane
// ---------------------------------------------------------------------------

constexpr int DPP_QUAD_XOR1 = 0xB1;
constexpr int DPP_QUAD_XOR2 = 0x4E;
constexpr int DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;
constexpr int DPP_ROW_NEWBCAST0 = 0x150;  // + lane: broadcast lane n of each row

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float row16_sum(float x) {
  x += dpp<DPP_QUAD_XOR1>(x);
  x += dpp<DPP_QUAD_XOR2>(x);
  x += dpp<DPP_ROW_HALF_MIRROR>(x);
  x += dpp<DPP_ROW_MIRROR>(x);
  return x;
}

__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, dpp<DPP_QUAD_XOR1>(x));
  x = fmaxf(x, dpp<DPP_QUAD_XOR2>(x));
  x = fmaxf(x, dpp<DPP_ROW_HALF_MIRROR>(x));
  x = fmaxf(x, dpp<DPP_ROW_MIRROR>(x));
  return x;
}

// x of this lane and x of lane ^ 32, without the LDS round trip of a
// ds_bpermute shuffle: v_permlane32_swap exchanges the two 32-lane halves of a
// register, so the pair (first, second) holds (x of lanes 0-31, x of lanes
// 32-63) in every lane. Max and sum over the pair are exact / commutative, so
// they equal x op shfl_xor(x, 32) bit for bit.
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// 2^x on the hardware exp unit (v_exp_f32). exp2(-inf) = 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;

}  // namespace skv

// ---------------------------------------------------------------------------
// Host-side error reporting shared by every C entry point.
// ---------------------------------------------------------------------------
namespace skv {
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

// Causal fp32 attention over a [B, T_cap, Hkv, D] key/value layout, query
// row i of sequence b at position start[b] + i (flash_fp32.hip).
int attn_fwd_f32(float* out, float* L, float* M, const float* q, const float* k, const float* v,
                 const int32_t* start, const int32_t* n_new, int B, int C, int Hq, int Hkv, int D,
                 int T_cap, float scale, hipStream_t s, const char* fn);

// The flash backward's kernels past a head dim of 128 (flash_fp32.hip built
// as its own translation unit with SKV_FLASH_WIDE_BWD; arguments checked by
// skv_flash_bwd). DP: the padded head dim (192 or 256), mode: its load mode.
int fbwd_wide(float* dq, float* dk, float* dv, const float* q, const float* k, const float* v,
              const float* o, const float* L, const float* M, const float* dout, float* delta,
              int B, int N, int H, int D, float scale, int DP, int mode, hipStream_t s);

// skv_linear over more than 64 rows: the tiled MFMA GEMM (gemm.hip). stats:
// M * 2 floats of workspace, used when ln_gamma is set.
int gemm_linear(float* y, const float* x, const float* w_t, const float* bias,
                const float* residual, const float* ln_gamma, const float* ln_beta, float ln_eps,
                int M, int N, int K, int activation, int split_cols, float* stats,
                hipStream_t s);
}  // namespace skv

#define SKV_REQUIRE(cond, code, ...)                          \
  do {                                                        \
    if (!(cond)) return ::skv::set_error((code), __VA_ARGS__); \
  } while (0)
