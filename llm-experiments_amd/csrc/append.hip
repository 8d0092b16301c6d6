// K/V append into the preallocated cache: a coalesced strided store.
//
// Reference behaviour: kv_cache_update (simple-llm/src/gpu/gpu_kv_cache.py:113-186)
// drives create_kv_cache_update_kernel (simple-llm/src/gpu/gpu_kernels.py:2725-2798),
// which copies new_k[b, :] to k_cache[(b*T_cap + pos)*E + :] for every b.
//
// Design: one workgroup per sequence for the single-token append. Each lane
// moves 16 bytes per tensor per iteration (a whole E = H_kv*D row is 1-8 KB),
// and after a workgroup barrier lane 0 advances lens[b]; no other workgroup
// touches lens[b], so the position update is race free and the whole decode
// step stays on the device. The reference takes any head_dim
// (gpu_kv_cache.py:55-64 checks only > 0): rows whose E is not a multiple of
// 8 elements (not 16-byte aligned in every dtype) move one element per lane
// and iteration instead.
#include "skv_common.h"

namespace skv {
namespace {

template <typename TI>
struct In16;  // 16 bytes of input converted to fp32
template <>
struct In16<float> {
  static constexpr int N = 4;
  __device__ __forceinline__ static void load(const float* p, float* o) {
    float4 x = *reinterpret_cast<const float4*>(p);
    o[0] = x.x; o[1] = x.y; o[2] = x.z; o[3] = x.w;
  }
};
template <>
struct In16<uint16_t> {
  static constexpr int N = 8;
  __device__ __forceinline__ static void load(const uint16_t* p, float* o) {
    uint4 x = *reinterpret_cast<const uint4*>(p);
    uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) { o[2 * i] = bf16w_lo(w[i]); o[2 * i + 1] = bf16w_hi(w[i]); }
  }
};

// One element in the cache's type: fp32 -> bf16 rounds to nearest even,
// bf16 -> fp32 is exact, equal types copy the bits.
template <typename TC, typename TI>
__device__ __forceinline__ TC convert_elem(TI x) {
  if constexpr (sizeof(TC) == sizeof(TI)) return x;
  else if constexpr (sizeof(TC) == 2) return f32_to_bf16(x);
  else return bf16_to_f32(x);
}

// Copy (TI == TC) keeps the input bits; fp32 -> bf16 rounds to nearest even;
// bf16 -> fp32 is exact. VEC: n is a multiple of 8 and both rows are 16-byte
// aligned (16-byte vectors); otherwise one element per lane and iteration.
template <typename TC, typename TI, bool VEC>
__device__ __forceinline__ void copy_row(TC* __restrict__ dst, const TI* __restrict__ src, int n,
                                         int tid, int nthreads) {
  if constexpr (!VEC) {
    for (int i = tid; i < n; i += nthreads) dst[i] = convert_elem<TC, TI>(src[i]);
  } else if constexpr (sizeof(TC) == sizeof(TI)) {
    // same type: move raw 16-byte vectors
    const uint4* s = reinterpret_cast<const uint4*>(src);
    uint4* d = reinterpret_cast<uint4*>(dst);
    const int nv = n * (int)sizeof(TC) / 16;
    for (int i = tid; i < nv; i += nthreads) d[i] = s[i];
  } else {
    constexpr int V = In16<TI>::N;
    for (int i = tid * V; i < n; i += nthreads * V) {
      float f[V];
      In16<TI>::load(src + i, f);
#pragma unroll
      for (int e = 0; e < V; ++e) {
        if constexpr (sizeof(TC) == 2) dst[i + e] = f32_to_bf16(f[e]);
        else dst[i + e] = f[e];
      }
    }
  }
}

template <typename TC, typename TI, bool PAGED, bool VEC>
__global__ __launch_bounds__(256) void k_append_one(TC* __restrict__ kc, TC* __restrict__ vc,
                                                    const TI* __restrict__ kn,
                                                    const TI* __restrict__ vn,
                                                    int32_t* __restrict__ lens,
                                                    const int32_t* __restrict__ block_table,
                                                    int max_blocks, int bs_shift, int E,
                                                    int T_cap) {
  const int b = blockIdx.x;
  const int pos = lens[b];
  // PAGED: capacity is max_blocks << bs_shift tokens.
  const int cap = PAGED ? (max_blocks << bs_shift) : T_cap;
  if (pos < 0 || pos >= cap) return;  // full (or corrupt): write nothing
  size_t row;
  if constexpr (PAGED) {
    const int blk = block_table[(size_t)b * max_blocks + (pos >> bs_shift)];
    row = ((size_t)blk << bs_shift) + (pos & ((1 << bs_shift) - 1));
  } else {
    row = (size_t)b * T_cap + pos;
  }
  const size_t src = (size_t)b * E;
  copy_row<TC, TI, VEC>(kc + row * E, kn + src, E, threadIdx.x, blockDim.x);
  copy_row<TC, TI, VEC>(vc + row * E, vn + src, E, threadIdx.x, blockDim.x);
  __syncthreads();  // every lane has read lens[b] before it moves
  if (threadIdx.x == 0) lens[b] = pos + 1;
}

// V consecutive elements of a row from src (one 16-byte load) into dst, in
// dst's type: one 16-byte store, two for bf16 -> fp32, one 8-byte store for
// fp32 -> bf16 (round to nearest even).
template <typename TC, typename TI>
__device__ __forceinline__ void copy_vec(TC* __restrict__ dst, const TI* __restrict__ src) {
  if constexpr (sizeof(TC) == sizeof(TI)) {
    *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
  } else {
    constexpr int V = In16<TI>::N;
    float f[V];
    In16<TI>::load(src, f);
    if constexpr (sizeof(TC) == 2) {
      *reinterpret_cast<uint2*>(dst) =
          make_uint2((uint32_t)f32_to_bf16(f[0]) | ((uint32_t)f32_to_bf16(f[1]) << 16),
                     (uint32_t)f32_to_bf16(f[2]) | ((uint32_t)f32_to_bf16(f[3]) << 16));
    } else {
#pragma unroll
      for (int e = 0; e < V; e += 4)
        *reinterpret_cast<float4*>(dst + e) = make_float4(f[e], f[e + 1], f[e + 2], f[e + 3]);
    }
  }
}

// Chunk append: grid (tiles of C * E / V threads, B), one 16-byte input
// vector of K and one of V per thread, so every load of the grid is in
// flight at once. (Four rows per workgroup in a loop, with 2-byte stores for
// fp32 -> bf16, took 16 us for C4's 50 MB chunk, 3.1 TB/s, on MI355X.)
// Rows i < n_new[b] of sequence b go to position lens[b] + i. lens is read
// only.
// NV = 2 (fp32 input into a bf16 cache): two 16-byte input vectors per
// thread, so the 8 bf16 results go out as one 16-byte store.
template <typename TC, typename TI, int NV = 1>
__global__ __launch_bounds__(256) void k_append_chunk(TC* __restrict__ kc, TC* __restrict__ vc,
                                                      const TI* __restrict__ kn,
                                                      const TI* __restrict__ vn,
                                                      const int32_t* __restrict__ lens,
                                                      const int32_t* __restrict__ n_new, int C,
                                                      int E, int T_cap) {
  static_assert(NV == 1 || (sizeof(TC) == 2 && sizeof(TI) == 4), "pairs: fp32 -> bf16 only");
  constexpr int V = In16<TI>::N * NV;  // elements per thread
  const int b = blockIdx.y;
  const int nv = E / V;           // thread slots per row
  const int g = blockIdx.x * 256 + threadIdx.x;
  const int r = g / nv, e = (g - r * nv) * V;
  const int n = n_new ? min(n_new[b], C) : C;
  const int pos = lens[b] + r;
  if (r >= n || pos < 0 || pos >= T_cap) return;
  const size_t dst = ((size_t)b * T_cap + pos) * E + e;
  const size_t src = ((size_t)b * C + r) * E + e;
  if constexpr (NV == 2) {
    auto pack8 = [](TC* d, const float* sp) {
      float f[8];
      In16<float>::load(sp, f);
      In16<float>::load(sp + 4, f + 4);
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = (uint32_t)f32_to_bf16(f[2 * i]) | ((uint32_t)f32_to_bf16(f[2 * i + 1]) << 16);
      *reinterpret_cast<uint4*>(d) = make_uint4(w[0], w[1], w[2], w[3]);
    };
    pack8(kc + dst, reinterpret_cast<const float*>(kn + src));
    pack8(vc + dst, reinterpret_cast<const float*>(vn + src));
  } else {
    copy_vec<TC, TI>(kc + dst, kn + src);
    copy_vec<TC, TI>(vc + dst, vn + src);
  }
}

// Chunk append of rows whose E is not a multiple of 8: grid (tiles of C * E
// threads, B), one element of K and one of V per thread.
template <typename TC, typename TI>
__global__ __launch_bounds__(256) void k_append_chunk_elem(TC* __restrict__ kc,
                                                           TC* __restrict__ vc,
                                                           const TI* __restrict__ kn,
                                                           const TI* __restrict__ vn,
                                                           const int32_t* __restrict__ lens,
                                                           const int32_t* __restrict__ n_new,
                                                           int C, int E, int T_cap) {
  const int b = blockIdx.y;
  const int g = blockIdx.x * 256 + threadIdx.x;
  const int r = g / E, e = g - r * E;
  const int n = n_new ? min(n_new[b], C) : C;
  const int pos = lens[b] + r;
  if (r >= n || pos < 0 || pos >= T_cap) return;
  const size_t dst = ((size_t)b * T_cap + pos) * E + e;
  const size_t src = ((size_t)b * C + r) * E + e;
  kc[dst] = convert_elem<TC, TI>(kn[src]);
  vc[dst] = convert_elem<TC, TI>(vn[src]);
}

__global__ void k_advance(int32_t* __restrict__ lens, const int32_t* __restrict__ n_new,
                          int n_const, int B, int T_cap) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const int n = n_new ? n_new[b] : n_const;
  lens[b] = min(lens[b] + n, T_cap);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int log2_exact(int x) {
  if (x <= 0 || (x & (x - 1))) return -1;
  int s = 0;
  while ((1 << s) < x) ++s;
  return s;
}

template <bool PAGED>
int launch_append_one(void* kc, void* vc, const void* kn, const void* vn, int32_t* lens,
                      const int32_t* bt, int max_blocks, int bs_shift, int B, int E, int T_cap,
                      int cache_dt, int in_dt, hipStream_t s) {
  dim3 grid(B), block(256);
  const bool vec = E % 8 == 0 && aligned16(kc) && aligned16(vc) && aligned16(kn) && aligned16(vn);
#define SKV_APPEND_CASE(TC, TI)                                                                   \
  do {                                                                                            \
    if (vec)                                                                                      \
      hipLaunchKernelGGL((k_append_one<TC, TI, PAGED, true>), grid, block, 0, s, (TC*)kc,         \
                         (TC*)vc, (const TI*)kn, (const TI*)vn, lens, bt, max_blocks, bs_shift, E, \
                         T_cap);                                                                  \
    else                                                                                          \
      hipLaunchKernelGGL((k_append_one<TC, TI, PAGED, false>), grid, block, 0, s, (TC*)kc,        \
                         (TC*)vc, (const TI*)kn, (const TI*)vn, lens, bt, max_blocks, bs_shift, E, \
                         T_cap);                                                                  \
  } while (0)
  if (cache_dt == SKV_F32 && in_dt == SKV_F32) SKV_APPEND_CASE(float, float);
  else if (cache_dt == SKV_F32 && in_dt == SKV_BF16) SKV_APPEND_CASE(float, uint16_t);
  else if (cache_dt == SKV_BF16 && in_dt == SKV_F32) SKV_APPEND_CASE(uint16_t, float);
  else SKV_APPEND_CASE(uint16_t, uint16_t);
#undef SKV_APPEND_CASE
  return check_launch("skv_append");
}

bool dt_ok(int dt) { return dt == SKV_F32 || dt == SKV_BF16; }

}  // namespace
}  // namespace skv

using namespace skv;

extern "C" int skv_append(void* k_cache, void* v_cache, const void* k_new, const void* v_new,
                          int32_t* lens, int B, int H_kv, int D, int T_cap, int cache_dt,
                          int in_dt, skv_stream_t stream) {
  SKV_REQUIRE(k_cache && v_cache && k_new && v_new && lens, SKV_E_INVALID,
              "skv_append: null pointer argument");
  SKV_REQUIRE(B > 0 && H_kv > 0 && D > 0 && T_cap > 0, SKV_E_INVALID,
              "skv_append: dims must be > 0 (B=%d H_kv=%d D=%d T_cap=%d)", B, H_kv, D, T_cap);
  SKV_REQUIRE(dt_ok(cache_dt) && dt_ok(in_dt), SKV_E_INVALID, "skv_append: bad dtype");
  return launch_append_one<false>(k_cache, v_cache, k_new, v_new, lens, nullptr, 0, 0, B,
                                  H_kv * D, T_cap, cache_dt, in_dt, (hipStream_t)stream);
}

extern "C" int skv_append_paged(void* k_pool, void* v_pool, const void* k_new, const void* v_new,
                                int32_t* lens, const int32_t* block_table, int max_blocks,
                                int block_size, int B, int H_kv, int D, int cache_dt, int in_dt,
                                skv_stream_t stream) {
  SKV_REQUIRE(k_pool && v_pool && k_new && v_new && lens && block_table, SKV_E_INVALID,
              "skv_append_paged: null pointer argument");
  SKV_REQUIRE(B > 0 && H_kv > 0 && D > 0 && max_blocks > 0, SKV_E_INVALID,
              "skv_append_paged: dims must be > 0");
  const int shift = log2_exact(block_size);
  SKV_REQUIRE(shift >= 0, SKV_E_INVALID, "skv_append_paged: block_size=%d not a power of two",
              block_size);
  SKV_REQUIRE(dt_ok(cache_dt) && dt_ok(in_dt), SKV_E_INVALID, "skv_append_paged: bad dtype");
  return launch_append_one<true>(k_pool, v_pool, k_new, v_new, lens, block_table, max_blocks,
                                 shift, B, H_kv * D, 0, cache_dt, in_dt, (hipStream_t)stream);
}

extern "C" int skv_append_chunk(void* k_cache, void* v_cache, const void* k_new,
                                const void* v_new, const int32_t* lens, const int32_t* n_new,
                                int B, int C, int H_kv, int D, int T_cap, int cache_dt, int in_dt,
                                skv_stream_t stream) {
  SKV_REQUIRE(k_cache && v_cache && k_new && v_new && lens, SKV_E_INVALID,
              "skv_append_chunk: null pointer argument");
  SKV_REQUIRE(B > 0 && C > 0 && H_kv > 0 && D > 0 && T_cap > 0, SKV_E_INVALID,
              "skv_append_chunk: dims must be > 0");
  SKV_REQUIRE(dt_ok(cache_dt) && dt_ok(in_dt), SKV_E_INVALID, "skv_append_chunk: bad dtype");
  const int E = H_kv * D;
  SKV_REQUIRE((size_t)C * E < (1u << 31), SKV_E_UNSUPPORTED, "skv_append_chunk: chunk too large");
  // 16-byte vectors when every row is 16-byte aligned in both dtypes
  const bool vec = E % 8 == 0 && aligned16(k_cache) && aligned16(v_cache) && aligned16(k_new) &&
                   aligned16(v_new);
  // fp32 rows into a bf16 cache: 8 elements a thread (E % 8 == 0 here)
  const bool pairs = vec && in_dt == SKV_F32 && cache_dt == SKV_BF16;
  const int V = vec ? (in_dt == SKV_BF16 || pairs ? 8 : 4) : 1;  // elements per thread
  dim3 grid((unsigned)(((size_t)C * (E / V) + 255) / 256), B), block(256);
  hipStream_t s = (hipStream_t)stream;
#define SKV_CHUNK_CASE(TC, TI)                                                                  \
  do {                                                                                          \
    if (vec)                                                                                    \
      hipLaunchKernelGGL((k_append_chunk<TC, TI>), grid, block, 0, s, (TC*)k_cache,             \
                         (TC*)v_cache, (const TI*)k_new, (const TI*)v_new, lens, n_new, C, E,   \
                         T_cap);                                                                \
    else                                                                                        \
      hipLaunchKernelGGL((k_append_chunk_elem<TC, TI>), grid, block, 0, s, (TC*)k_cache,        \
                         (TC*)v_cache, (const TI*)k_new, (const TI*)v_new, lens, n_new, C, E,   \
                         T_cap);                                                                \
  } while (0)
  if (cache_dt == SKV_F32 && in_dt == SKV_F32) SKV_CHUNK_CASE(float, float);
  else if (cache_dt == SKV_F32 && in_dt == SKV_BF16) SKV_CHUNK_CASE(float, uint16_t);
  else if (pairs)
    hipLaunchKernelGGL((k_append_chunk<uint16_t, float, 2>), grid, block, 0, s,
                       (uint16_t*)k_cache, (uint16_t*)v_cache, (const float*)k_new,
                       (const float*)v_new, lens, n_new, C, E, T_cap);
  else if (cache_dt == SKV_BF16 && in_dt == SKV_F32) SKV_CHUNK_CASE(uint16_t, float);
  else SKV_CHUNK_CASE(uint16_t, uint16_t);
#undef SKV_CHUNK_CASE
  return check_launch("skv_append_chunk");
}

extern "C" int skv_advance(int32_t* lens, const int32_t* n_new, int n_const, int B, int T_cap,
                           skv_stream_t stream) {
  SKV_REQUIRE(lens && B > 0 && T_cap > 0, SKV_E_INVALID, "skv_advance: bad arguments");
  hipLaunchKernelGGL(k_advance, dim3((B + 255) / 256), dim3(256), 0, (hipStream_t)stream, lens,
                     n_new, n_const, B, T_cap);
  return check_launch("skv_advance");
}
