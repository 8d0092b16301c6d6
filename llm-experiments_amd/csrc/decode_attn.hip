// Cached single-query decode attention on gfx950: the head dims 64 and 128
// (pass-1 kernels tuned per shape), the merge pass for every head dim, and
// the C entry points. Kernel design: decode_kernels.h; pass 1 for any other
// head dim: decode_attn_generic.hip.
#include <algorithm>
#include <atomic>
#include <mutex>

#include "decode_kernels.h"

namespace skv {
namespace {

using dec::heads_per_group;
using dec::kNumCUs;

// Online merge of pieces st, st + NS, st + 2 NS, ... of one stream, loading
// the partials of U pieces per memory round trip (k_decode_merge).
template <int U, int NS, int D, int EPL, bool MASK>
__device__ __forceinline__ void merge_pieces(const float* __restrict__ ws_o,
                                             const float* __restrict__ ws_ml, size_t base,
                                             int np, int st, int li, float& M, float& L,
                                             float (&O)[EPL], int RS) {
  for (int n0 = st; n0 < np; n0 += U * NS) {
    float mn[U], ln[U], on[U][EPL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t pn = base + min(n0 + u * NS, np - 1);
      const float2 ml = *reinterpret_cast<const float2*>(ws_ml + pn * 2);
      mn[u] = ml.x;
      ln[u] = ml.y;
      const float* src = ws_o + pn * RS + li * EPL;
      if constexpr (MASK) {  // elements past the head dim: clamped, never stored
#pragma unroll
        for (int e = 0; e < EPL; ++e) on[u][e] = ws_o[pn * RS + min(li * EPL + e, RS - 1)];
      } else if constexpr (EPL == 4) {
        const float4 x = *reinterpret_cast<const float4*>(src);
        on[u][0] = x.x; on[u][1] = x.y; on[u][2] = x.z; on[u][3] = x.w;
      } else {
#pragma unroll
        for (int e = 0; e < EPL; ++e) on[u][e] = src[e];
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      // every piece holds at least one token, so mn is finite; piece u = 0 is
      // always valid (n0 < np), so M is finite for every later u
      const bool ok = n0 + u * NS < np;
      const float Mn = ok ? fmaxf(M, mn[u]) : M;
      const float wa = ok ? fast_exp2(M - Mn) : 1.f;
      const float wb = ok ? fast_exp2(mn[u] - Mn) : 0.f;
      L = L * wa + ln[u] * wb;
#pragma unroll
      for (int e = 0; e < EPL; ++e) O[e] = O[e] * wa + on[u][e] * wb;
      M = Mn;
    }
  }
}

// Pass 2: grid (Hq, B), 256 threads = NS piece streams x 256/NS lanes; lane
// i of a stream owns elements [i*EPL, (i+1)*EPL), EPL = D*NS/256 (8 streams
// of 32 lanes up to a head dim of 256, 2 streams of 128 lanes past it).
// Sequence b's pieces are the slots w + b for the workgroups w its token
// range [cum[b], cum[b+1]) overlaps. Each stream merges pieces n = stream,
// stream + NS, ... online; the NS streams merge in LDS.
template <int D, bool MASK, int NS = 8>
__global__ __launch_bounds__(256) void k_decode_merge(void* __restrict__ out, int out_dt,
                                                      const long long* __restrict__ cum,
                                                      const float* __restrict__ ws_o,
                                                      const float* __restrict__ ws_ml, int Hq,
                                                      int chunk, int n_wg, int n_slots,
                                                      int32_t* __restrict__ lens_inc, int cap,
                                                      int Dr) {
  constexpr int LS = 256 / NS;  // lanes per stream
  constexpr int EPL = D / LS;
  static_assert(EPL * LS == D, "the padded head dim splits evenly over a stream's lanes");
  const int RS = MASK ? Dr : D;  // head dim (D is its padded size when MASK)
  const int hq = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  // fused append: the sequence's length moves past its new token once pass 1
  // (which read it) has finished; nothing below reads lens
  if (lens_inc && hq == 0 && tid == 0) {
    const int p = lens_inc[b];
    if (p >= 0 && p < cap) lens_inc[b] = p + 1;
  }
  const int st = tid / LS, li = tid % LS;
  const size_t obase = ((size_t)b * Hq + hq) * RS;
  const long long c0 = cum[b], c1 = cum[b + 1];
  if (c1 <= c0) {
    for (int d = tid; d < RS; d += 256) store_elem(out, obase + d, out_dt, 0.f);
    return;
  }
  if (c1 > (long long)n_wg * chunk) {  // plan too small for these lengths: flag, never read past it
    for (int d = tid; d < RS; d += 256) store_elem(out, obase + d, out_dt, __builtin_nanf(""));
    return;
  }
  const long long wf = c0 / chunk;
  const int np = (int)((c1 - 1) / chunk - wf + 1);
  const size_t base = (size_t)hq * n_slots + wf + b;
  float M = -INFINITY, L = 0.f, O[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) O[e] = 0.f;
  // Stream st merges pieces st, st + NS, st + 2 NS, ... in that order. The
  // partials of U pieces are loaded together, at indices clamped to the last
  // piece (in bounds), so one memory round trip serves U pieces. The merge
  // step has no branch: a clamped copy past np gets weights 1 (state) and 0
  // (its finite values), an exact no-op. (With a bounds check per piece the
  // compiler moved each piece's loads behind its check, one round trip per
  // piece.)
  // Streams with more than two pieces take 8 per round trip; shorter
  // sequences (C1: at most two per stream) take 2, which measured 1.2 us per
  // step faster there than loading 8 clamped copies (np is uniform in the
  // workgroup, so the branch is too).
  // (Past a head dim of 256, EPL is 4 to 16 floats: U = 2 keeps the loads of
  // a round trip within a lane's registers.)
  constexpr int UL = EPL > 8 ? 2 : 8;
  if (np > 2 * NS) merge_pieces<UL, NS, D, EPL, MASK>(ws_o, ws_ml, base, np, st, li, M, L, O, RS);
  else merge_pieces<2, NS, D, EPL, MASK>(ws_o, ws_ml, base, np, st, li, M, L, O, RS);
  __shared__ float sm_ml[NS][2];
  __shared__ float sm_o[NS][D];
  if (li == 0) {
    sm_ml[st][0] = M;
    sm_ml[st][1] = L;
  }
#pragma unroll
  for (int e = 0; e < EPL; ++e) sm_o[st][li * EPL + e] = O[e];
  __syncthreads();
  float MM = -INFINITY;
#pragma unroll
  for (int s = 0; s < NS; ++s) MM = fmaxf(MM, sm_ml[s][0]);
  for (int d = tid; d < RS; d += 256) {
    float LL = 0.f, OO = 0.f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const float w = fast_exp2(sm_ml[s][0] - MM);  // streams with no piece: w = 0
      LL = fmaf(w, sm_ml[s][1], LL);
      OO = fmaf(w, sm_o[s][d], OO);
    }
    store_elem(out, obase + d, out_dt, OO / LL);
  }
}

template <typename TC, int D, int G, bool PAGED>
void launch_partial(const DecodeArgs& a, hipStream_t s) {
  // Tokens per row per iteration: 8 x 16 B (or 8 x 8 B for bf16 D=64) in
  // flight per lane for K and as many for V; 4 x 32 B for fp32 D=128; and
  // 4 x 16 B for bf16 D=128 without GQA, which the plan runs at one
  // workgroup per CU on long streams: C4 158.8 -> 155.5 us per call on
  // MI355X (8 tokens in flight: 82.9% of 8 TB/s, 4: 84.6%).
  // Without GQA at D = 64 (C2, C3: short pieces of 32-token chunks) groups of
  // 4 tokens with the prefetching loop, for both cache types: against 8-token
  // groups (prefetching fp32, single-set bf16), C3 598.5 against 605.1 us per
  // step with the fp32 cache and 543.3 against 545.1 with bf16, C2 19.6
  // against 20.1 us per call (two rounds on one MI355X); 2-token groups and
  // 16-token groups were slower.
  constexpr bool kMha64 = D == 64 && G == 1;
  constexpr bool kMhaBf16 = sizeof(TC) == 2 && D == 128 && G == 1;
  constexpr int TPG = ((sizeof(TC) == 4 && D == 128) || kMhaBf16 || kMha64) ? 4 : 8;
  // Load prefetch across token groups (a second register set) for fp32
  // caches without GQA: C2/C3 measured 2-3 % faster per call on MI355X; the
  // bf16 C4 case measured 1 % slower (occupancy 4 -> 2), so it keeps one set.
  constexpr bool PF = (G == 1 && sizeof(TC) == 4) || kMha64;
  launch_partial_t<TC, D, G, TPG, PAGED, PF, 1, false>(a, s);
}

// Pass 1: grouped queries over a bf16 cache on the matrix cores
// (decode_gqa_mfma.hip), else D = 64 or 128 (this file) or any other D <= 256
// (the masked kernels of decode_attn_generic.hip).
template <typename TC, bool PAGED>
int dispatch_partial(const DecodeArgs& a, int D, int G, hipStream_t s) {
  if (dec::gqa_mfma_eligible(a, G, sizeof(TC) == 2, PAGED))
    return dec::launch_partial_gqa(a, G, PAGED, s);
#define SKV_DEC(DD, GG)                                    \
  if (D == DD && G == GG) {                                \
    launch_partial<TC, DD, GG, PAGED>(a, s);               \
    return 0;                                              \
  }
  SKV_DEC(64, 1) SKV_DEC(64, 2) SKV_DEC(64, 4) SKV_DEC(64, 8)
  SKV_DEC(128, 1) SKV_DEC(128, 2) SKV_DEC(128, 4) SKV_DEC(128, 8)
#undef SKV_DEC
  return PAGED ? dec::launch_partial_generic_paged(a, G, sizeof(TC) == 2, s)
               : dec::launch_partial_generic(a, G, sizeof(TC) == 2, s);
}

// Workspace layout of a call: fp32 partials o [Hq][n_slots][D], then (m, l)
// [Hq][n_slots][2], then B + 1 int64 prefix sums; each part starts 16-byte
// aligned (odd head dims would misalign the (m, l) pairs and the int64s).
struct WsLayout {
  size_t o_floats, ml_floats, bytes;
};
WsLayout ws_layout(int B, int Hq, int D, int n_chunks_max) {
  const size_t parts = (size_t)B * Hq * n_chunks_max;
  WsLayout w;
  w.o_floats = (parts * D + 3) / 4 * 4;
  w.ml_floats = (parts * 2 + 3) / 4 * 4;
  w.bytes = (w.o_floats + w.ml_floats) * sizeof(float) + (size_t)(B + 1) * sizeof(long long);
  return w;
}

// Padded head dim of the masked kernels: a power of two in [32, 2048].
int padded_dim(int D) {
  int p = 32;
  while (p < D) p <<= 1;
  return p;
}

bool dt_ok(int dt) { return dt == SKV_F32 || dt == SKV_BF16; }

int log2_exact(int x) {
  if (x <= 0 || (x & (x - 1))) return -1;
  int s = 0;
  while ((1 << s) < x) ++s;
  return s;
}

template <bool PAGED>
int decode_common(void* out, const void* q, const void* k, const void* v, const int32_t* lens,
                  const int32_t* bt, int max_blocks, int block_size, int B, int Hq, int Hkv,
                  int D, int T_cap, float scale, int chunk, int n_chunks_max, void* ws,
                  size_t ws_bytes, int cache_dt, int q_dt, int out_dt, hipStream_t s,
                  const void* new_k = nullptr, const void* new_v = nullptr, int in_dt = 0,
                  const char* name = nullptr) {
  const bool app = new_k != nullptr;
  const char* fn = name ? name
                        : app ? (PAGED ? "skv_append_decode_attn_paged" : "skv_append_decode_attn")
                              : (PAGED ? "skv_decode_attn_paged" : "skv_decode_attn");
  SKV_REQUIRE(!app || (new_v && dt_ok(in_dt)), SKV_E_INVALID,
              "%s: new_v missing or bad input dtype", fn);
  SKV_REQUIRE(out && q && k && v && lens && ws, SKV_E_INVALID, "%s: null pointer argument", fn);
  SKV_REQUIRE(!PAGED || bt, SKV_E_INVALID, "%s: null block table", fn);
  SKV_REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && D > 0, SKV_E_INVALID, "%s: dims must be > 0", fn);
  SKV_REQUIRE(B <= 65535, SKV_E_UNSUPPORTED, "%s: B=%d exceeds the grid limit", fn, B);
  SKV_REQUIRE(PAGED || T_cap > 0, SKV_E_INVALID, "%s: T_cap must be > 0", fn);
  SKV_REQUIRE(Hq % Hkv == 0, SKV_E_INVALID, "%s: H_q=%d not a multiple of H_kv=%d", fn, Hq, Hkv);
  SKV_REQUIRE(Hq % Hkv != 0 || D <= dec::max_head_dim(Hq / Hkv), SKV_E_UNSUPPORTED,
              "%s: head_dim %d with %d query heads per kv head (supported: 1 to %d)", fn, D,
              Hq / Hkv, dec::max_head_dim(Hq / Hkv));
  SKV_REQUIRE(dt_ok(cache_dt) && dt_ok(q_dt) && dt_ok(out_dt), SKV_E_INVALID, "%s: bad dtype",
              fn);
  SKV_REQUIRE(chunk > 0 && chunk % 16 == 0, SKV_E_INVALID,
              "%s: chunk_tokens=%d must be a positive multiple of 16", fn, chunk);
  SKV_REQUIRE(n_chunks_max >= 2 && n_chunks_max <= (1 << 20), SKV_E_INVALID,
              "%s: n_chunks_max=%d out of range [2, 2^20]", fn, n_chunks_max);
  const long long n_slots = (long long)B * n_chunks_max;
  SKV_REQUIRE(n_slots <= (1LL << 31) - 1, SKV_E_UNSUPPORTED,
              "%s: B * n_chunks_max = %lld exceeds the grid limit", fn, n_slots);
  const size_t need = skv_decode_workspace_bytes(B, Hq, D, n_chunks_max);
  SKV_REQUIRE(ws_bytes >= need, SKV_E_WORKSPACE, "%s: workspace %zu bytes < %zu required", fn,
              ws_bytes, need);
  int shift = 0;
  if (PAGED) {
    shift = log2_exact(block_size);
    SKV_REQUIRE(shift >= 0, SKV_E_INVALID, "%s: block_size=%d not a power of two", fn,
                block_size);
    SKV_REQUIRE(max_blocks > 0 && (long)max_blocks << shift < (1L << 31), SKV_E_INVALID,
                "%s: max_blocks=%d out of range", fn, max_blocks);
  }
  DecodeArgs a;
  a.q = q; a.k = k; a.v = v; a.lens = lens; a.block_table = bt;
  a.max_blocks = max_blocks; a.bs_shift = shift;
  a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.T_cap = T_cap; a.D = D;
  a.cap = PAGED ? (max_blocks << shift) : T_cap;
  a.qscale = scale * LOG2E;
  a.chunk = chunk; a.q_dt = q_dt;
  // B pieces more than workgroups: a sequence can start inside a workgroup.
  a.n_slots = (int)n_slots;
  a.n_wg = (int)(n_slots - B);
  a.hw = heads_per_group(Hkv);
  a.S = kMaxRows / a.hw;
  SKV_REQUIRE(Hkv / a.hw <= 65535, SKV_E_UNSUPPORTED, "%s: H_kv=%d exceeds the grid limit", fn,
              Hkv);
  const WsLayout wl = ws_layout(B, Hq, D, n_chunks_max);
  a.ws_o = static_cast<float*>(ws);
  a.ws_ml = a.ws_o + wl.o_floats;
  a.cum = reinterpret_cast<long long*>(a.ws_ml + wl.ml_floats);
  a.new_k = new_k;
  a.new_v = new_v;
  a.in_dt = in_dt;
  const int G = Hq / Hkv;
  int rc = cache_dt == SKV_BF16 ? dispatch_partial<uint16_t, PAGED>(a, D, G, s)
                                : dispatch_partial<float, PAGED>(a, D, G, s);
  if (rc) return rc;
  rc = check_launch(fn);
  if (rc) return rc;
  int32_t* lens_inc = app ? const_cast<int32_t*>(lens) : nullptr;
#define SKV_MERGE(DD, MM)                                                                      \
  hipLaunchKernelGGL((k_decode_merge<DD, MM>), dim3(Hq, B), dim3(256), 0, s, out, out_dt, a.cum, \
                     a.ws_o, a.ws_ml, Hq, chunk, a.n_wg, a.n_slots, lens_inc, a.cap, D)
#define SKV_MERGE_WIDE(DD)                                                                       \
  hipLaunchKernelGGL((k_decode_merge<DD, true, 2>), dim3(Hq, B), dim3(256), 0, s, out, out_dt,    \
                     a.cum, a.ws_o, a.ws_ml, Hq, chunk, a.n_wg, a.n_slots, lens_inc, a.cap, D)
  const int DP = padded_dim(D);
  if (D == 64) SKV_MERGE(64, false);
  else if (D == 128) SKV_MERGE(128, false);
  else if (DP == 32) SKV_MERGE(32, true);
  else if (DP == 64) SKV_MERGE(64, true);
  else if (DP == 128) SKV_MERGE(128, true);
  else if (DP == 256) SKV_MERGE(256, true);
  else if (DP == 512) SKV_MERGE_WIDE(512);
  else if (DP == 1024) SKV_MERGE_WIDE(1024);
  else SKV_MERGE_WIDE(2048);
#undef SKV_MERGE
#undef SKV_MERGE_WIDE
  return check_launch(fn);
}

// ---------------------------------------------------------------------------
// Scratch of skv_decode_attn_noalloc: the split-K workspace in a file-scope
// device array, kScratchBytes per GPU for the life of the process. Host code
// never uses the array's name as an address (on the host it is only a
// handle): the device address comes from hipGetSymbolAddress, queried once
// per device with that device current, and kept here.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = SKV_DECODE_NOALLOC_MAX_BYTES;
__device__ __align__(256) unsigned char scratch[kScratchBytes];
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of this GPU's scratch (the current device's).
int scratch_ptr(void** out, const char* fn) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(SKV_E_HIP, "%s: hipGetDevice: %s", fn, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(SKV_E_UNSUPPORTED, "%s: device %d beyond the %d this library serves", fn, dev,
                     kMaxDevices);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));  // `dev` is the current device
      if (e != hipSuccess || p == nullptr)
        return set_error(SKV_E_HIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", fn, dev,
                         hipGetErrorString(e));
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return SKV_OK;
}

}  // namespace
}  // namespace skv

using namespace skv;

extern "C" int skv_decode_plan(int B, int H_q, int H_kv, int head_dim, int cache_dtype,
                               int max_len, long long total_len, int chunk_hint, int* chunk_tokens,
                               int* n_chunks_max) {
  SKV_REQUIRE(chunk_tokens && n_chunks_max, SKV_E_INVALID, "skv_decode_plan: null output");
  SKV_REQUIRE(B > 0 && H_q > 0 && H_kv > 0 && max_len > 0, SKV_E_INVALID,
              "skv_decode_plan: dims must be > 0 (B=%d H_q=%d H_kv=%d max_len=%d)", B, H_q, H_kv,
              max_len);
  SKV_REQUIRE(H_q % H_kv == 0, SKV_E_INVALID,
              "skv_decode_plan: H_q=%d is not a multiple of H_kv=%d", H_q, H_kv);
  int chunk;
  const long long tot = total_len > 0 ? total_len : (long long)B * max_len;
  const int G = H_q / H_kv;
  if (chunk_hint > 0) {
    chunk = (int)(((long)chunk_hint + 15) / 16 * 16);
  } else if (cache_dtype == SKV_BF16 && (head_dim == 64 || head_dim == 128) &&
             (G == 2 || G == 4 || G == 8)) {
    // The matrix-core GQA kernel (decode_gqa_mfma.hip): one workgroup of 8
    // wavefronts per CU, kv heads in groups of up to 8. It is bound by HBM,
    // which served fewer concurrent streams than CUs faster. C5 (132K
    // tokens, 8 kv heads), one process, chunk sizes interleaved over three
    // rounds: 252 workgroups 97.8 us per call, 231: 96.1-96.6, 219-225:
    // 95.1-95.5, 208: 95.9, 189: 98.2, 173: 104.3; past 256 (512 tokens:
    // 258) a second round of workgroups costs 45%.
    int hw = 1;
    while (hw < 8 && H_kv % (hw * 2) == 0) hw *= 2;
    const long long groups = H_kv / hw;
    const long long target = kNumCUs * 7 / 8;
    long long per = (tot * groups + target - 1) / target;
    per = (per + 15) / 16 * 16;
    chunk = (int)std::min<long long>(std::max<long long>(per, 32), 8192);
  } else {
    // About 512 busy workgroups per call: two per CU on MI355X's 256 CUs.
    // Grids that leave some CUs one workgroup more than others (e.g. 336
    // workgroups) or that use more, shorter chunks measured 5-15% slower on
    // C4 (4 x 32K tokens). A workgroup owns chunk tokens of the flat token
    // stream (every sequence's filled tokens end to end), so the chunk
    // follows the batch's total fill and a ragged batch splits as evenly as
    // a uniform one. Chunks are 32 to 8192 tokens.
    // Without grouped queries (H_q == H_kv) a workgroup does little VALU
    // work per byte, and one workgroup per CU with twice the chunk streams
    // faster once chunks are long: C4 161.6 -> 159.5 us per call (256 ->
    // 512 tokens), as a plain non-temporal read of K and V does (87.3% ->
    // 89.5% of 8 TB/s). With grouped queries the VALU kernels' per-wavefront
    // exp and dot work needs the second workgroup (C5: 119 -> 159 us per
    // call at one per CU).
    const long long groups = H_kv / heads_per_group(H_kv);
    long long target = 2 * kNumCUs;
    if (H_q == H_kv && (tot * groups + kNumCUs - 1) / kNumCUs >= 256) target = kNumCUs;
    long long per = (tot * groups + target - 1) / target;
    per = (per + 31) / 32 * 32;
    if (per < 32) per = 32;
    if (per > 8192) per = 8192;
    chunk = (int)per;
  }
  // ceil(max_len / chunk) workgroups per sequence cover B * max_len tokens;
  // one more slot per sequence holds the piece of a sequence that starts
  // inside a workgroup's range.
  const long n = ((long)max_len + chunk - 1) / chunk + 1;
  SKV_REQUIRE(n <= (1 << 20), SKV_E_UNSUPPORTED,
              "skv_decode_plan: %ld chunks exceed the grid limit", n);
  *chunk_tokens = chunk;
  *n_chunks_max = (int)n;
  return SKV_OK;
}

extern "C" size_t skv_decode_workspace_bytes(int B, int H_q, int D, int n_chunks_max) {
  if (B <= 0 || H_q <= 0 || D <= 0 || n_chunks_max <= 0) return 0;
  // partials (o[D], m, l) per (query head, slot), then B + 1 int64 prefix sums
  return ws_layout(B, H_q, D, n_chunks_max).bytes;
}

extern "C" int skv_decode_attn(void* out, const void* q, const void* k_cache, const void* v_cache,
                               const int32_t* lens, int B, int H_q, int H_kv, int D, int T_cap,
                               float scale, int chunk_tokens, int n_chunks_max, void* ws,
                               size_t ws_bytes, int cache_dt, int q_dt, int out_dt,
                               skv_stream_t stream) {
  return decode_common<false>(out, q, k_cache, v_cache, lens, nullptr, 0, 0, B, H_q, H_kv, D,
                              T_cap, scale, chunk_tokens, n_chunks_max, ws, ws_bytes, cache_dt,
                              q_dt, out_dt, (hipStream_t)stream);
}

extern "C" int skv_decode_attn_paged(void* out, const void* q, const void* k_pool,
                                     const void* v_pool, const int32_t* lens,
                                     const int32_t* block_table, int max_blocks, int block_size,
                                     int B, int H_q, int H_kv, int D, float scale,
                                     int chunk_tokens, int n_chunks_max, void* ws,
                                     size_t ws_bytes, int cache_dt, int q_dt, int out_dt,
                                     skv_stream_t stream) {
  return decode_common<true>(out, q, k_pool, v_pool, lens, block_table, max_blocks, block_size, B,
                             H_q, H_kv, D, 0, scale, chunk_tokens, n_chunks_max, ws, ws_bytes,
                             cache_dt, q_dt, out_dt, (hipStream_t)stream);
}

extern "C" int skv_append_decode_attn(void* out, const void* q, void* k_cache, void* v_cache,
                                      const void* new_k, const void* new_v, int32_t* lens, int B,
                                      int H_q, int H_kv, int D, int T_cap, float scale,
                                      int chunk_tokens, int n_chunks_max, void* ws,
                                      size_t ws_bytes, int cache_dt, int in_dt, int q_dt,
                                      int out_dt, skv_stream_t stream) {
  if (!new_k)
    return set_error(SKV_E_INVALID, "skv_append_decode_attn: null pointer argument");
  return decode_common<false>(out, q, k_cache, v_cache, lens, nullptr, 0, 0, B, H_q, H_kv, D,
                              T_cap, scale, chunk_tokens, n_chunks_max, ws, ws_bytes, cache_dt,
                              q_dt, out_dt, (hipStream_t)stream, new_k, new_v, in_dt);
}

extern "C" int skv_append_decode_attn_paged(void* out, const void* q, void* k_pool, void* v_pool,
                                            const void* new_k, const void* new_v, int32_t* lens,
                                            const int32_t* block_table, int max_blocks,
                                            int block_size, int B, int H_q, int H_kv, int D,
                                            float scale, int chunk_tokens, int n_chunks_max,
                                            void* ws, size_t ws_bytes, int cache_dt, int in_dt,
                                            int q_dt, int out_dt, skv_stream_t stream) {
  if (!new_k)
    return set_error(SKV_E_INVALID, "skv_append_decode_attn_paged: null pointer argument");
  return decode_common<true>(out, q, k_pool, v_pool, lens, block_table, max_blocks, block_size, B,
                             H_q, H_kv, D, 0, scale, chunk_tokens, n_chunks_max, ws, ws_bytes,
                             cache_dt, q_dt, out_dt, (hipStream_t)stream, new_k, new_v, in_dt);
}

extern "C" int skv_decode_attn_noalloc(void* out, const void* q, const void* k_cache,
                                       const void* v_cache, const int32_t* lens, int B, int H_q,
                                       int H_kv, int D, int T_cap, float scale, int chunk_tokens,
                                       int n_chunks_max, int cache_dt, int q_dt, int out_dt,
                                       skv_stream_t stream) {
  const char* fn = "skv_decode_attn_noalloc";
  if (B > 0 && H_q > 0 && D > 0 && n_chunks_max > 0) {
    const size_t need = skv_decode_workspace_bytes(B, H_q, D, n_chunks_max);
    SKV_REQUIRE(need <= kScratchBytes, SKV_E_WORKSPACE,
                "%s: this plan needs %zu bytes of split-K scratch, above the %zu-byte maximum "
                "(call skv_decode_attn with a workspace instead)",
                fn, need, kScratchBytes);
  }
  void* ws = nullptr;
  const int rc = scratch_ptr(&ws, fn);
  if (rc) return rc;
  return decode_common<false>(out, q, k_cache, v_cache, lens, nullptr, 0, 0, B, H_q, H_kv, D,
                              T_cap, scale, chunk_tokens, n_chunks_max, ws, kScratchBytes,
                              cache_dt, q_dt, out_dt, (hipStream_t)stream, nullptr, nullptr, 0,
                              fn);
}
