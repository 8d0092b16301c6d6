// Direct single-query decode attention with the step's append: the
// workgroups of one (sequence, head) read that head's whole filled row and
// write the output themselves, with no merge pass. The fill is NOT
// advanced: the caller advances it (the model's step does so at the start of
// the next step, in skv_next_embed), which is what lets the workgroups of one
// sequence run without knowing of each other. The same semantics as
// skv_append_decode_attn otherwise (gpu_kv_cache.py:194-289,
// gpu_kernels.py:2801-2938): new_k/new_v[b] goes to position lens[b] (if
// lens[b] in [0, cap)), then
//   o = softmax(scale * q . K[t], t <= lens[b]) . V
// over the filled rows and the new one; a negative fill is an empty row.
//
// Split S (1, 2 or 4): a (sequence, head) gets S workgroups of 64 / S rows of
// 16 lanes (1024 threads in all), workgroup s taking the s-th of S equal
// parts of the row, so a batch of few (sequence, head) pairs spreads over S
// times as many CUs (a long row is otherwise read at one CU's return rate).
// Row r of a workgroup takes tokens r, r + R, r + 2R, ... of its part; lane
// i of a row owns elements [i*D/16, (i+1)*D/16) of each K and V row it reads
// (16 or 32 bytes for fp32, 8 or 16 for bf16). A row issues the loads of TOK
// tokens before using any, sums the q.k partials over its 16 lanes with DPP,
// and keeps an online softmax (m in log2 units, l, o). The new token is
// folded in by row 0 of the last part's workgroup from registers (rounded to
// the cache precision, as the stored copy), and stored to the cache by the
// same row. The rows of a workgroup merge in LDS in row order. With S > 1
// each workgroup then writes its (m, l, o) as device-scope atomic stores
// (they write through to memory: no L2 write-back fence is needed), counts
// its arrival on the (sequence, head)'s counter, and the last to arrive
// reads all S partials back (device-scope atomic loads, served from memory),
// merges them in part order, writes the output and puts the counter back to
// zero. Results are bitwise reproducible and do not depend on which
// workgroup arrives last.
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
  float* part;     // S > 1: [B * H][S][D + 2] partials (o[D], m, l)
  unsigned* cnt;   // S > 1: [B * H] arrival counters, zero between calls
};

constexpr int kDirRows = 64;  // rows of 16 lanes per (sequence, head), over its S workgroups
// The workspace starts with a fixed block of arrival counters, one per
// (sequence, head), and the partials follow at a fixed offset: calls of any
// shape can share one workspace without a call's partials landing on
// another's counters.
constexpr int kDirCounters = 65536;
constexpr size_t kDirCounterBytes = kDirCounters * sizeof(unsigned);

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

template <typename TC, int D, int TOK, int S>
__global__ __launch_bounds__(kDirRows * 16 / S) void k_decode_direct(DirectArgs a) {
  constexpr int EPL = D / 16;
  constexpr int R = kDirRows / S;  // rows of this workgroup
  // (sequence, head, part) from the flat workgroup index, the sequence
  // slowest. The dispatcher deals workgroups in index order over the XCDs and
  // their CUs, so indices 256 apart share a CU; with the sequence fastest
  // (B = 16) those were parts of one sequence, and the CUs that drew a long
  // row got all of its bytes. Sequence slowest, a CU's workgroups come from
  // different sequences (C3, 16 ragged rows, fp32 cache, S = 4: 543.4 ->
  // 528.7 us per decode step on MI355X, same output bits). B * H * S <= 2^31
  // (checked on the host).
  const unsigned wid = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  const int part = (int)(wid % S), h = (int)((wid / S) % (unsigned)a.H),
            b = (int)(wid / (S * (unsigned)a.H));
  const int tid = threadIdx.x, row = tid >> 4, ln = tid & 15;
  const int p = a.lens[b];
  const int Lc = min(max(p, 0), a.T_cap);  // cached rows of the sequence
  // this workgroup's part [t_lo, t_hi) of the cached rows
  const int per = (Lc + S - 1) / S;
  const int t_lo = min(part * per, Lc), t_hi = min(t_lo + per, Lc);
  const bool app = a.new_k != nullptr && p >= 0 && p < a.T_cap && part == S - 1;  // uniform
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
  for (int t0 = t_lo + row; t0 < t_hi; t0 += R * TOK) {
    float kx[TOK][EPL], vx[TOK][EPL];
#pragma unroll
    for (int j = 0; j < TOK; ++j) {  // every load first; rows past the part reread its last
      const size_t off = base + (size_t)min(t0 + j * R, t_hi - 1) * rs;
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
      s[j] = t0 + j * R < t_hi ? d : -INFINITY;
      smax = fmaxf(smax, s[j]);
    }
    const float mn = fmaxf(m, smax);  // finite: token t0 < t_hi is valid
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
  // merge the workgroup's rows in row order
  __shared__ float s_m[R], s_l[R];
  __shared__ float s_o[R][D];
  if (ln == 0) {
    s_m[row] = m;
    s_l[row] = l;
  }
#pragma unroll
  for (int e = 0; e < EPL; ++e) s_o[row][ln * EPL + e] = o[e];
  __syncthreads();
  float M = -INFINITY, LL = 0.f, OO = 0.f;
  if (tid < D) {
    for (int r = 0; r < R; ++r) M = fmaxf(M, s_m[r]);
    if (M != -INFINITY) {
      for (int r = 0; r < R; ++r) {
        const float w = fast_exp2(s_m[r] - M);  // rows with no token: 0
        LL = fmaf(w, s_l[r], LL);
        OO = fmaf(w, s_o[r][tid], OO);
      }
    }
  }
  const size_t oi = ((size_t)b * a.H + h) * D + tid;
  if constexpr (S > 1) {
    // this part's (o, m, l) out to memory, then the last of the S to arrive merges
    __shared__ unsigned s_last;
    const size_t bh = (size_t)b * a.H + h;
    float* pp = a.part + (bh * S + part) * (D + 2);
    if (tid < D) {
      __hip_atomic_store(pp + tid, OO, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (tid == 0) {
        __hip_atomic_store(pp + D, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(pp + D + 1, LL, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);  // the write-through stores are acknowledged
    __syncthreads();
    if (tid == 0)
      s_last = __hip_atomic_fetch_add(a.cnt + bh, 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(S - 1);
    __syncthreads();
    if (!s_last) return;
    if (tid == 0) __hip_atomic_store(a.cnt + bh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid >= D) return;
    const float* pb = a.part + bh * S * (D + 2);
    float pm[S], pl[S], po[S];
#pragma unroll
    for (int z = 0; z < S; ++z) {  // every part's loads in flight together
      po[z] = __hip_atomic_load(pb + z * (D + 2) + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      pm[z] = __hip_atomic_load(pb + z * (D + 2) + D, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      pl[z] = __hip_atomic_load(pb + z * (D + 2) + D + 1, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
    }
    M = -INFINITY;
#pragma unroll
    for (int z = 0; z < S; ++z) M = fmaxf(M, pm[z]);
    LL = 0.f;
    OO = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int z = 0; z < S; ++z) {  // part order: the bits do not depend on the arrival order
        const float w = fast_exp2(pm[z] - M);  // parts with no token: 0
        LL = fmaf(w, pl[z], LL);
        OO = fmaf(w, po[z], OO);
      }
    }
  }
  // an empty row (no cached token, no append) gives 0, as the split kernels
  if (tid < D) store_elem(a.out, oi, a.out_dt, LL > 0.f ? OO / LL : 0.f);
}

template <typename TC, int D>
void launch_direct(const DirectArgs& a, int S, hipStream_t s) {
  // tokens in flight per row: 4 at D = 128 (64 registers of K and V a lane;
  // 16 wavefronts a CU leave 128); at D = 64, 8 on one workgroup per row and
  // 4 on split rows (C3, S = 4, whole generate runs on MI355X: fp32 cache
  // 22,652 tokens/s at 4 against 22,540 at 8, 22,614 at 2, 22,504 at 6,
  // 21,385 at 12; bf16 cache 24,493-24,503 at 4 against 24,165-24,172 at 8)
  constexpr int TOK1 = D == 64 ? 8 : 4, TOKS = 4;
  const dim3 grid(a.B, a.H, S);
  if (S == 1) hipLaunchKernelGGL((k_decode_direct<TC, D, TOK1, 1>), grid, dim3(kDirRows * 16), 0, s, a);
  else if (S == 2) hipLaunchKernelGGL((k_decode_direct<TC, D, TOKS, 2>), grid, dim3(kDirRows * 8), 0, s, a);
  else hipLaunchKernelGGL((k_decode_direct<TC, D, TOKS, 4>), grid, dim3(kDirRows * 4), 0, s, a);
}

}  // namespace
}  // namespace skv

using namespace skv;

extern "C" size_t skv_decode_direct_workspace_bytes(int B, int H, int D, int n_split) {
  if (B <= 0 || H <= 0 || D <= 0 || n_split <= 1) return 0;
  // the arrival counters' fixed block, then the partials
  return kDirCounterBytes + (size_t)B * H * n_split * (D + 2) * sizeof(float);
}

extern "C" int skv_append_decode_attn_direct(void* out, const void* q, void* k_cache,
                                             void* v_cache, const void* new_k,
                                             const void* new_v, const int32_t* lens, int B,
                                             int H, int D, int T_cap, float scale,
                                             int cache_dtype, int in_dtype, int q_dtype,
                                             int out_dtype, int n_split, void* ws,
                                             size_t ws_bytes, skv_stream_t stream) {
  const char* fn = "skv_append_decode_attn_direct";
  SKV_REQUIRE(out && q && k_cache && v_cache && new_k && new_v && lens, SKV_E_INVALID,
              "%s: null pointer argument", fn);
  SKV_REQUIRE(B > 0 && H > 0 && T_cap > 0, SKV_E_INVALID, "%s: dims must be > 0", fn);
  SKV_REQUIRE(B <= 65535 && H <= 65535 && (long)B * H * 4 <= 2147483647L, SKV_E_UNSUPPORTED,
              "%s: grid too large", fn);
  SKV_REQUIRE(D == 64 || D == 128, SKV_E_UNSUPPORTED, "%s: D=%d (supported: 64, 128)", fn, D);
  SKV_REQUIRE((cache_dtype == SKV_F32 || cache_dtype == SKV_BF16) &&
                  (in_dtype == SKV_F32 || in_dtype == SKV_BF16) &&
                  (q_dtype == SKV_F32 || q_dtype == SKV_BF16) &&
                  (out_dtype == SKV_F32 || out_dtype == SKV_BF16),
              SKV_E_INVALID, "%s: bad dtype", fn);
  SKV_REQUIRE(n_split == 1 || n_split == 2 || n_split == 4, SKV_E_INVALID,
              "%s: n_split=%d (supported: 1, 2, 4)", fn, n_split);
  // the cache rows are read as 16-byte (fp32) or 8-byte (bf16) vectors
  const uintptr_t al = cache_dtype == SKV_F32 ? 15 : 7;
  SKV_REQUIRE((((uintptr_t)k_cache | (uintptr_t)v_cache) & al) == 0, SKV_E_UNSUPPORTED,
              "%s: k_cache and v_cache must be %d-byte aligned for this cache dtype", fn,
              (int)al + 1);
  SKV_REQUIRE(n_split == 1 || (long)B * H <= kDirCounters, SKV_E_UNSUPPORTED,
              "%s: B * H = %ld above the %d (sequence, head) rows a split call takes", fn,
              (long)B * H, kDirCounters);
  const size_t need = skv_decode_direct_workspace_bytes(B, H, D, n_split);
  SKV_REQUIRE(n_split == 1 || (ws && ws_bytes >= need && ((uintptr_t)ws & 3) == 0),
              SKV_E_WORKSPACE, "%s: workspace %zu bytes < %zu required (4-byte aligned)", fn,
              ws_bytes, need);
  DirectArgs a{out, q, k_cache, v_cache, new_k, new_v, lens, B, H, T_cap,
               scale * 1.4426950408889634f, q_dtype, in_dtype, out_dtype, nullptr, nullptr};
  if (n_split > 1) {
    a.cnt = static_cast<unsigned*>(ws);
    a.part = reinterpret_cast<float*>(static_cast<char*>(ws) + kDirCounterBytes);
  }
  hipStream_t s = (hipStream_t)stream;
  if (cache_dtype == SKV_F32) {
    if (D == 64) launch_direct<float, 64>(a, n_split, s);
    else launch_direct<float, 128>(a, n_split, s);
  } else {
    if (D == 64) launch_direct<uint16_t, 64>(a, n_split, s);
    else launch_direct<uint16_t, 128>(a, n_split, s);
  }
  return check_launch(fn);
}
