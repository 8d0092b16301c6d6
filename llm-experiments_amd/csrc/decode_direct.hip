// Direct single-query decode attention with the step's append: one workgroup
// per (sequence, head) reads that head's whole filled row and writes the
// output itself, with no split over the token stream, no partials and no
// merge pass. The fill is NOT advanced: the caller advances it (the model's
// step does so at the start of the next step, in skv_next_embed), which is
// what lets the workgroups of one sequence run without knowing of each
// other. The same semantics as skv_append_decode_attn otherwise
// (gpu_kv_cache.py:194-289, gpu_kernels.py:2801-2938): new_k/new_v[b] goes
// to position lens[b] (if lens[b] in [0, cap)), then
//   o = softmax(scale * q . K[t], t <= lens[b]) . V
// over the filled rows and the new one; a negative fill is an empty row.
//
// Workgroup of 1024 threads = 64 rows of 16 lanes. Row r takes tokens
// r, r + 64, r + 128, ... of the head's row; lane i of a row owns elements
// [i*D/16, (i+1)*D/16) of each K and V row it reads (16 or 32 bytes for
// fp32, 8 or 16 for bf16). A row issues the loads of TOK tokens before
// using any (up to 64 * TOK tokens in flight per workgroup: one workgroup
// per CU streams near a CU's return rate), sums the q.k partials over its
// 16 lanes with DPP, and keeps an online softmax (m in log2 units, l, o).
// The new token is folded in by row 0 from registers (rounded to the cache
// precision, as the stored copy), and stored to the cache by the same row.
// The 64 rows merge in LDS in row order: results are bitwise reproducible.
#include "skv_common.h"

namespace skv {
namespace {

struct DirectArgs {
  void* out;
  const void* q;
  void* k;
  void* v;
  const void* new_k;  // NULL: no append
  const void* new_v;
  const int32_t* lens;
  int B, H, T_cap;
  float qscale;  // softmax scale * log2(e)
  int q_dt, in_dt, out_dt;
};

constexpr int kDirRows = 64;
constexpr int kDirThreads = kDirRows * 16;

template <typename TC>
__device__ __forceinline__ float cache_round(float x) {
  if constexpr (sizeof(TC) == 2) return bf16_to_f32(f32_to_bf16(x));
  else return x;
}

// EPL elements of a cache row at element offset i (16-byte vectors for fp32,
// 8- or 16-byte for bf16).
template <typename TC, int EPL>
__device__ __forceinline__ void load_row(const TC* p, float (&x)[EPL]) {
  if constexpr (sizeof(TC) == 4) {
#pragma unroll
    for (int j = 0; j < EPL / 4; ++j) {
      const float4 a = reinterpret_cast<const float4*>(p)[j];
      x[4 * j] = a.x; x[4 * j + 1] = a.y; x[4 * j + 2] = a.z; x[4 * j + 3] = a.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < EPL / 4; ++j) {
      const uint2 a = reinterpret_cast<const uint2*>(p)[j];
      x[4 * j] = bf16w_lo(a.x); x[4 * j + 1] = bf16w_hi(a.x);
      x[4 * j + 2] = bf16w_lo(a.y); x[4 * j + 3] = bf16w_hi(a.y);
    }
  }
}

template <typename TC, int D, int TOK>
__global__ __launch_bounds__(kDirThreads) void k_decode_direct(DirectArgs a) {
  constexpr int EPL = D / 16;
  const int b = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, row = tid >> 4, ln = tid & 15;
  const int p = a.lens[b];
  const int L = min(max(p, 0), a.T_cap);                        // cached rows read
  const bool app = a.new_k != nullptr && p >= 0 && p < a.T_cap;  // uniform
  const size_t qo = ((size_t)b * a.H + h) * D + ln * EPL;
  float q[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) q[e] = load_elem(a.q, qo + e, a.q_dt) * a.qscale;
  const TC* kc = static_cast<const TC*>(a.k);
  const TC* vc = static_cast<const TC*>(a.v);
  const size_t rs = (size_t)a.H * D;                                   // token stride
  const size_t base = (size_t)b * a.T_cap * rs + (size_t)h * D + ln * EPL;
  float m = -INFINITY, l = 0.f, o[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) o[e] = 0.f;
  for (int t0 = row; t0 < L; t0 += kDirRows * TOK) {
    float kx[TOK][EPL], vx[TOK][EPL];
#pragma unroll
    for (int j = 0; j < TOK; ++j) {  // every load first; rows past L reread row L - 1
      const size_t off = base + (size_t)min(t0 + j * kDirRows, L - 1) * rs;
      load_row<TC, EPL>(kc + off, kx[j]);
      load_row<TC, EPL>(vc + off, vx[j]);
    }
    float s[TOK], smax = -INFINITY;
#pragma unroll
    for (int j = 0; j < TOK; ++j) {
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) d = fmaf(q[e], kx[j][e], d);
      d = row16_sum(d);
      s[j] = t0 + j * kDirRows < L ? d : -INFINITY;
      smax = fmaxf(smax, s[j]);
    }
    const float mn = fmaxf(m, smax);  // finite: token t0 < L is valid
    const float al = fast_exp2(m - mn);
    l *= al;
#pragma unroll
    for (int e = 0; e < EPL; ++e) o[e] *= al;
#pragma unroll
    for (int j = 0; j < TOK; ++j) {
      const float w = fast_exp2(s[j] - mn);  // 0 for a masked token
      l += w;
#pragma unroll
      for (int e = 0; e < EPL; ++e) o[e] = fmaf(w, vx[j][e], o[e]);
    }
    m = mn;
  }
  if (app && row == 0) {  // the new token: stored, and folded in from registers
    const size_t no = ((size_t)b * a.H + h) * D + ln * EPL;
    float nk[EPL], nv[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      nk[e] = cache_round<TC>(load_elem(a.new_k, no + e, a.in_dt));
      nv[e] = cache_round<TC>(load_elem(a.new_v, no + e, a.in_dt));
    }
    const size_t off = base + (size_t)p * rs;
    TC* kw = static_cast<TC*>(a.k);
    TC* vw = static_cast<TC*>(a.v);
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      store_elem(kw, off + e, sizeof(TC) == 2 ? SKV_BF16 : SKV_F32, nk[e]);
      store_elem(vw, off + e, sizeof(TC) == 2 ? SKV_BF16 : SKV_F32, nv[e]);
    }
    float d = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) d = fmaf(q[e], nk[e], d);
    d = row16_sum(d);
    const float mn = fmaxf(m, d);
    const float al = fast_exp2(m - mn), w = fast_exp2(d - mn);  // m = -inf: al = 0
    l = l * al + w;
#pragma unroll
    for (int e = 0; e < EPL; ++e) o[e] = fmaf(w, nv[e], o[e] * al);
    m = mn;
  }
  // merge the 64 rows in row order
  __shared__ float s_m[kDirRows], s_l[kDirRows];
  __shared__ float s_o[kDirRows][D];
  if (ln == 0) {
    s_m[row] = m;
    s_l[row] = l;
  }
#pragma unroll
  for (int e = 0; e < EPL; ++e) s_o[row][ln * EPL + e] = o[e];
  __syncthreads();
  if (tid < D) {
    float M = -INFINITY;
    for (int r = 0; r < kDirRows; ++r) M = fmaxf(M, s_m[r]);
    float LL = 0.f, OO = 0.f;
    if (M != -INFINITY) {
      for (int r = 0; r < kDirRows; ++r) {
        const float w = fast_exp2(s_m[r] - M);  // rows with no token: 0
        LL = fmaf(w, s_l[r], LL);
        OO = fmaf(w, s_o[r][tid], OO);
      }
    }
    // an empty row (no cached token, no append) gives 0, as the split kernels
    store_elem(a.out, ((size_t)b * a.H + h) * D + tid, a.out_dt, LL > 0.f ? OO / LL : 0.f);
  }
}

template <typename TC, int D>
void launch_direct(const DirectArgs& a, hipStream_t s) {
  // tokens in flight per row: 8 at D = 64, 4 at D = 128 (64 registers of K
  // and V a lane; 16 wavefronts a CU leave 128)
  constexpr int TOK = D == 64 ? 8 : 4;
  hipLaunchKernelGGL((k_decode_direct<TC, D, TOK>), dim3(a.B, a.H), dim3(kDirThreads), 0, s, a);
}

}  // namespace
}  // namespace skv

using namespace skv;

extern "C" int skv_append_decode_attn_direct(void* out, const void* q, void* k_cache,
                                             void* v_cache, const void* new_k,
                                             const void* new_v, const int32_t* lens, int B,
                                             int H, int D, int T_cap, float scale,
                                             int cache_dtype, int in_dtype, int q_dtype,
                                             int out_dtype, skv_stream_t stream) {
  const char* fn = "skv_append_decode_attn_direct";
  SKV_REQUIRE(out && q && k_cache && v_cache && new_k && new_v && lens, SKV_E_INVALID,
              "%s: null pointer argument", fn);
  SKV_REQUIRE(B > 0 && H > 0 && T_cap > 0, SKV_E_INVALID, "%s: dims must be > 0", fn);
  SKV_REQUIRE(B <= 65535 && H <= 65535, SKV_E_UNSUPPORTED, "%s: grid too large", fn);
  SKV_REQUIRE(D == 64 || D == 128, SKV_E_UNSUPPORTED, "%s: D=%d (supported: 64, 128)", fn, D);
  SKV_REQUIRE((cache_dtype == SKV_F32 || cache_dtype == SKV_BF16) &&
                  (in_dtype == SKV_F32 || in_dtype == SKV_BF16) &&
                  (q_dtype == SKV_F32 || q_dtype == SKV_BF16) &&
                  (out_dtype == SKV_F32 || out_dtype == SKV_BF16),
              SKV_E_INVALID, "%s: bad dtype", fn);
  // the cache rows are read as 16-byte (fp32) or 8-byte (bf16) vectors
  const uintptr_t al = cache_dtype == SKV_F32 ? 15 : 7;
  SKV_REQUIRE((((uintptr_t)k_cache | (uintptr_t)v_cache) & al) == 0, SKV_E_UNSUPPORTED,
              "%s: k_cache and v_cache must be %d-byte aligned for this cache dtype", fn,
              (int)al + 1);
  DirectArgs a{out, q, k_cache, v_cache, new_k, new_v, lens, B, H, T_cap,
               scale * 1.4426950408889634f, q_dtype, in_dtype, out_dtype};
  hipStream_t s = (hipStream_t)stream;
  if (cache_dtype == SKV_F32) {
    if (D == 64) launch_direct<float, 64>(a, s);
    else launch_direct<float, 128>(a, s);
  } else {
    if (D == 64) launch_direct<uint16_t, 64>(a, s);
    else launch_direct<uint16_t, 128>(a, s);
  }
  return check_launch(fn);
}
