// Cached single-query decode attention: split-K (flash-decoding) on gfx950.
//
// Reference behaviour: attention_with_kv_cache
// (simple-llm/src/gpu/gpu_kv_cache.py:194-289) launches
// create_attention_with_kv_cache_kernel (simple-llm/src/gpu/gpu_kernels.py:2801-2938):
// per (b, h), s_t = scale * q . K[t] for t < len, softmax over [0, len),
// o = sum_t p_t V[t]. One workgroup per (b, h) and len <= 256 there.
//
// Design (HBM-bound GEMV, no MFMA):
//  * Pass 1, grid (workgroup, kv-head group). The sequences' filled tokens,
//    laid end to end, form one flat stream; workgroup w owns its tokens
//    [w*chunk, (w+1)*chunk), cut into pieces at sequence boundaries, for a
//    group of HW kv heads. Equal ranges keep a ragged batch as evenly spread
//    over the CUs as a uniform one. A workgroup is made of 16-lane DPP rows:
//    row r serves kv head r % HW of the group
//    and token substream r / HW (S substreams, HW*S <= 16). Lane i of a row
//    owns elements [i*D/16, (i+1)*D/16) of each K and V row it reads, as
//    16-byte (or 8-byte) vector loads. Because the cache is [B, T, H_kv, D],
//    the HW heads of one token are contiguous: a wavefront (4 rows) reads
//    4 consecutive head rows of the same token (1 KB for bf16 D=128), and
//    the workgroup sweeps whole token rows in address order. This keeps HBM
//    reads contiguous; reading one head's 256-byte rows at a 4 KB stride
//    measured ~11% slower on MI355X. The loads are non-temporal.
//  * The q.k partial dot is summed across the row with four DPP steps, so
//    every lane of the row holds every score and the online softmax
//    (running max m, sum l, accumulator o) needs no further cross-lane
//    traffic. Scores are in log2 units (log2(e) is folded into the query
//    scale) so each exp is a single v_exp_f32. GQA: a row serves all
//    G = H_q/H_kv query heads of its kv head, so each K/V byte is read once.
//  * Each (piece, query head) gets one partial (m, l, o[D]) in the
//    workspace. With S > 1 the S substreams of a head merge through LDS
//    first.
//  * Pass 2, grid (q_head, seq), 256 threads: log-sum-exp merge of the
//    sequence's piece partials, 8 streams in parallel, then across the
//    streams in LDS.
// No atomics anywhere: results are bitwise reproducible run to run.
#include "skv_common.h"

namespace skv {
namespace {

constexpr int kMaxRows = 16;  // DPP rows per workgroup (256 threads)
constexpr int kNumCUs = 256;  // compute units of an MI355X

struct DecodeArgs {
  const void* q;
  const void* k;
  const void* v;
  const int32_t* lens;
  const int32_t* block_table;
  int max_blocks;
  int bs_shift;
  int B, Hq, Hkv, T_cap;
  int cap;       // tokens a sequence can hold: T_cap, or max_blocks * block_size
  float qscale;  // softmax scale * log2(e)
  int chunk;     // tokens of the flat token stream per pass-1 workgroup
  int n_wg;      // pass-1 workgroups along the token stream
  int n_slots;   // partial slots per query head (>= n_wg + B - 1)
  int q_dt;
  int hw;        // kv heads per workgroup
  int S;         // token substreams per kv head
  long long* cum;  // [B + 1] exclusive prefix sums of the clamped lengths
  float* ws_o;   // [Hq][n_slots][D]
  float* ws_ml;  // [Hq][n_slots][2]  (m in log2 units, l)
  // Fused append (skv_append_decode_attn*): the token new_k/new_v[b] goes to
  // position lens[b] (if lens[b] in [0, cap)) before the attention, which
  // then covers it; NULL for plain decode attention.
  const void* new_k;  // [B, Hkv, D] of in_dt
  const void* new_v;
  int in_dt;
};

__device__ __forceinline__ bool appends(const DecodeArgs& a, int b) {
  return a.new_k != nullptr && a.lens[b] >= 0 && a.lens[b] < a.cap;
}

// Lengths outside [0, cap] are clamped so no row outside the cache (or block
// table entry outside the table) is ever addressed; a fused append adds its
// token.
__device__ __forceinline__ int clamped_len(const DecodeArgs& a, int b) {
  return min(max(a.lens[b], 0), a.cap) + (appends(a, b) ? 1 : 0);
}

// Stores the EPL values x (rounded to the cache's precision in place) at p.
template <typename TC, int EPL>
__device__ __forceinline__ void store_row(TC* p, float (&x)[EPL]) {
  if constexpr (sizeof(TC) == 4) {
#pragma unroll
    for (int i = 0; i < EPL / 4; ++i)
      *reinterpret_cast<float4*>(reinterpret_cast<float*>(p) + 4 * i) =
          make_float4(x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]);
  } else {
    uint32_t w[EPL / 2];
#pragma unroll
    for (int e = 0; e < EPL; e += 2) {
      const uint16_t lo = f32_to_bf16(x[e]), hi = f32_to_bf16(x[e + 1]);
      x[e] = bf16_to_f32(lo);
      x[e + 1] = bf16_to_f32(hi);
      w[e / 2] = (uint32_t)lo | ((uint32_t)hi << 16);
    }
    if constexpr (EPL == 8)
      *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
    else
      *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
  }
}

template <typename TC, int D, bool PAGED>
__device__ __forceinline__ const TC* row_ptr(const TC* base, const DecodeArgs& a, int b, int t,
                                             int hk) {
  size_t row;
  if constexpr (PAGED) {
    const int blk = a.block_table[(size_t)b * a.max_blocks + (t >> a.bs_shift)];
    row = ((size_t)blk << a.bs_shift) + (t & ((1 << a.bs_shift) - 1));
  } else {
    row = (size_t)b * a.T_cap + t;
  }
  return base + (row * a.Hkv + hk) * D;
}

// Position `first` of the flat token stream (the sequences' filled tokens
// laid end to end) -> (sequence, offset in it), or sequence -1 past the end.
// Rounds of blockDim sequences: an inclusive scan of the clamped lengths
// within each wavefront (shuffles, no barrier), then across the wavefronts
// through LDS. The workgroup with write_cum also stores the exclusive prefix
// sums (and the total at [B]) for the merge pass.
__device__ void locate(const DecodeArgs& a, long long first, bool write_cum, int* b_out,
                       int* off_out) {
  __shared__ long long s_wave[4];  // wavefront totals of one round (blockDim <= 256)
  __shared__ int s_b, s_off;
  const int tid = threadIdx.x, nt = blockDim.x, lane = tid & 63, wv = tid >> 6;
  const int nwaves = (nt + 63) >> 6;
  if (tid == 0) s_b = -1;
  long long carry = 0;
  for (int base = 0; base < a.B; base += nt) {
    const int bb = base + tid;
    const long long L = bb < a.B ? clamped_len(a, bb) : 0;
    long long x = L;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {  // lanes below are active, also in a partial wavefront
      const long long y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (lane == 63 || tid == nt - 1) s_wave[wv] = x;
    __syncthreads();
    long long incl = carry + x, round_total = 0;
    for (int w2 = 0; w2 < nwaves; ++w2) {
      const long long t = s_wave[w2];
      if (w2 < wv) incl += t;
      round_total += t;
    }
    const long long excl = incl - L;
    if (bb < a.B) {
      if (write_cum) a.cum[bb] = excl;
      if (L > 0 && excl <= first && first < incl) {  // exactly one thread
        s_b = bb;
        s_off = (int)(first - excl);
      }
    }
    carry += round_total;
    __syncthreads();
    if (!write_cum && s_b >= 0) break;  // uniform: read after the barrier
  }
  if (write_cum && tid == 0) a.cum[a.B] = carry;
  // Uniform values from LDS: readfirstlane keeps them (and the addresses
  // derived from them) in scalar registers.
  *b_out = __builtin_amdgcn_readfirstlane(s_b);
  *off_out = __builtin_amdgcn_readfirstlane(s_off);
}

// Tokens [start, end) of sequence b for the workgroup's kv heads -> one
// partial per query head at `slot`.
template <typename TC, int D, int G, int TPG, bool PAGED, bool PF>
__device__ __forceinline__ void decode_piece(const DecodeArgs& a, int hg, int b, int start,
                                             int end, int slot) {
  constexpr int EPL = D / 16;
  const int tid = threadIdx.x;
  const int rid = tid >> 4;  // DPP row
  const int li = tid & 15;   // lane within the row
  const int e0 = li * EPL;
  const int hl = rid % a.hw;  // kv head within the group
  const int sub = rid / a.hw; // token substream
  const int hk = hg * a.hw + hl;
  const int S = a.S;

  // With the prefetching loop (fp32 caches, G = 1) the query rows are loaded
  // as raw words, two vector loads per head without a branch on q's dtype
  // (for bf16 the second repeats the first), and converted and scaled only
  // after the first token group's K/V loads are issued: the q round trip then
  // overlaps the K/V one instead of preceding it (short pieces, as in a model
  // step). The other loops convert at once, which keeps one copy of q in
  // registers.
  const bool q_bf16 = a.q_dt == SKV_BF16;
  float q[G][EPL];
  uint32_t qraw[PF ? G : 1][EPL];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const size_t qoff = ((size_t)b * a.Hq + hk * G + h) * D + e0;
    if constexpr (PF) {
      const char* qp = static_cast<const char*>(a.q) + qoff * (q_bf16 ? 2 : 4);
      if constexpr (EPL == 8) {
        const u32x4_t w0 = *reinterpret_cast<const u32x4_t*>(qp);
        const u32x4_t w1 = *reinterpret_cast<const u32x4_t*>(q_bf16 ? qp : qp + 16);
        qraw[h][0] = w0.x; qraw[h][1] = w0.y; qraw[h][2] = w0.z; qraw[h][3] = w0.w;
        qraw[h][4] = w1.x; qraw[h][5] = w1.y; qraw[h][6] = w1.z; qraw[h][7] = w1.w;
      } else {  // D = 64
        const u32x2_t w0 = *reinterpret_cast<const u32x2_t*>(qp);
        const u32x2_t w1 = *reinterpret_cast<const u32x2_t*>(q_bf16 ? qp : qp + 8);
        qraw[h][0] = w0.x; qraw[h][1] = w0.y; qraw[h][2] = w1.x; qraw[h][3] = w1.y;
      }
    } else {
      if constexpr (EPL == 8)
        load8_f32(a.q, qoff, a.q_dt, q[h]);
      else  // D = 64
        load4_f32(a.q, qoff, a.q_dt, q[h]);
#pragma unroll
      for (int e = 0; e < EPL; ++e) q[h][e] *= a.qscale;
    }
  }
  auto ready_q = [&]() {  // the prefetching loop's deferred conversion
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float v = q_bf16 ? ((e & 1) ? bf16w_hi(qraw[h][e >> 1]) : bf16w_lo(qraw[h][e >> 1]))
                               : __uint_as_float(qraw[h][e]);
        q[h][e] = v * a.qscale;
      }
  };

  float m[G], l[G], acc[G][EPL];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[h][e] = 0.f;
  }

  const TC* kb = static_cast<const TC*>(a.k);
  const TC* vb = static_cast<const TC*>(a.v);
  const int step = S * TPG;
  // A fused append's token is the last of its sequence: the main loop stops
  // before it (mend) and substream 0 takes it from the input after the loop.
  const bool has_new = appends(a, b) && end == clamped_len(a, b);
  const int mend = has_new ? end - 1 : end;

  // Loads of the TPG tokens from t0 on (rows past end are clamped: masked in
  // consume, never out of bounds). FLOOR: also for t0 >= mend, where the rows
  // clamp to max(mend - 1, 0): a cached row, or (mend = 0: the piece holds
  // only an appended token) row 0, which that append is writing, so it exists.
#define SKV_LOAD_TILE_(KF, VF, T0, FLOOR)                                     \
  {                                                                           \
    _Pragma("unroll") for (int u = 0; u < TPG; ++u) {                         \
      int t_ = min((T0) + u, mend - 1);                                        \
      if (FLOOR) t_ = max(t_, 0);                                             \
      KF[u].load(row_ptr<TC, D, PAGED>(kb, a, b, t_, hk) + e0);               \
    }                                                                         \
    _Pragma("unroll") for (int u = 0; u < TPG; ++u) {                         \
      int t_ = min((T0) + u, mend - 1);                                        \
      if (FLOOR) t_ = max(t_, 0);                                             \
      VF[u].load(row_ptr<TC, D, PAGED>(vb, a, b, t_, hk) + e0);               \
    }                                                                         \
  }
#define SKV_LOAD_TILE(KF, VF, T0) SKV_LOAD_TILE_(KF, VF, T0, false)
  // Online softmax and PV of the TPG tokens from t0 held in KF, VF.
#define SKV_CONSUME(KF, VF, T0)                                               \
  {                                                                           \
    _Pragma("unroll") for (int h = 0; h < G; ++h) {                           \
      float s[TPG];                                                           \
      _Pragma("unroll") for (int u = 0; u < TPG; ++u) {                       \
        float d = 0.f;                                                        \
        _Pragma("unroll") for (int e = 0; e < EPL; ++e) d =                   \
            fmaf(q[h][e], KF[u].get(e), d);                                   \
        d = row16_sum(d);                                                     \
        s[u] = ((T0) + u < mend) ? d : -INFINITY;                              \
      }                                                                       \
      float mx = m[h];                                                        \
      _Pragma("unroll") for (int u = 0; u < TPG; ++u) mx = fmaxf(mx, s[u]);   \
      const float alpha = fast_exp2(m[h] - mx); /* 0 on the first tile */     \
      m[h] = mx;                                                              \
      float ls = 0.f;                                                         \
      _Pragma("unroll") for (int e = 0; e < EPL; ++e) acc[h][e] *= alpha;     \
      _Pragma("unroll") for (int u = 0; u < TPG; ++u) {                       \
        const float p = fast_exp2(s[u] - mx);                                 \
        ls += p;                                                              \
        _Pragma("unroll") for (int e = 0; e < EPL; ++e) acc[h][e] =           \
            fmaf(p, VF[u].get(e), acc[h][e]);                                 \
      }                                                                       \
      l[h] = l[h] * alpha + ls;                                               \
    }                                                                         \
  }

  if constexpr (PF) {
    // Two register sets: the loads of the next token group are in flight
    // while the current one is consumed (one HBM round trip per piece
    // instead of one per group).
    Frag<TC, EPL> ka[TPG], va[TPG], kn[TPG], vn[TPG];
    int t0 = start + sub * TPG;
    // The first group is loaded unconditionally (rows floored, unused when
    // t0 >= mend): behind a branch, the join before q's conversion made the
    // compiler wait for every load issued, the K/V ones included.
    SKV_LOAD_TILE_(ka, va, t0, true);
    __builtin_amdgcn_sched_barrier(0);  // the conversion stays after these loads
    ready_q();
    while (t0 < mend) {
      if (t0 + step < mend) SKV_LOAD_TILE(kn, vn, t0 + step);
      SKV_CONSUME(ka, va, t0);
      t0 += step;
      if (t0 >= mend) break;
      if (t0 + step < mend) SKV_LOAD_TILE(ka, va, t0 + step);
      SKV_CONSUME(kn, vn, t0);
      t0 += step;
    }
  } else {
    for (int t0 = start + sub * TPG; t0 < mend; t0 += step) {
      Frag<TC, EPL> kf[TPG], vf[TPG];
      SKV_LOAD_TILE(kf, vf, t0);
      SKV_CONSUME(kf, vf, t0);
    }
  }
#undef SKV_CONSUME
#undef SKV_LOAD_TILE
#undef SKV_LOAD_TILE_

  if (has_new && sub == 0) {
    // The appended token: the input row, rounded to the cache's precision,
    // is stored at position end - 1 and attended like the cached ones.
    const int tn = end - 1;
    float kx[EPL], vx[EPL];
    const size_t src = ((size_t)b * a.Hkv + hk) * D + e0;
    if constexpr (EPL == 8) {
      load8_f32(a.new_k, src, a.in_dt, kx);
      load8_f32(a.new_v, src, a.in_dt, vx);
    } else {
      load4_f32(a.new_k, src, a.in_dt, kx);
      load4_f32(a.new_v, src, a.in_dt, vx);
    }
    store_row<TC, EPL>(const_cast<TC*>(row_ptr<TC, D, PAGED>(kb, a, b, tn, hk)) + e0, kx);
    store_row<TC, EPL>(const_cast<TC*>(row_ptr<TC, D, PAGED>(vb, a, b, tn, hk)) + e0, vx);
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) d = fmaf(q[h][e], kx[e], d);
      d = row16_sum(d);
      const float mx = fmaxf(m[h], d);
      const float alpha = fast_exp2(m[h] - mx);  // 0 if the row saw no token yet
      const float p = fast_exp2(d - mx);
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[h][e] = fmaf(p, vx[e], acc[h][e] * alpha);
      l[h] = l[h] * alpha + p;
      m[h] = mx;
    }
  }

  if (S == 1) {
    // One row per head: it holds the whole piece's partial. A row that saw no
    // token (only possible if the piece is shorter than TPG) keeps m = -inf,
    // l = 0, o = 0.
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const size_t pidx = (size_t)(hk * G + h) * a.n_slots + slot;
#pragma unroll
      for (int e = 0; e < EPL; ++e) a.ws_o[pidx * D + e0 + e] = acc[h][e];
      if (li == 0) {
        a.ws_ml[pidx * 2 + 0] = m[h];
        a.ws_ml[pidx * 2 + 1] = l[h];
      }
    }
    return;
  }

  // S > 1: merge the S substreams of each head through LDS, one query head
  // at a time. Rows that saw no token drop out through exp2(-inf) = 0.
  __shared__ float sm_ml[kMaxRows][2];
  __shared__ float sm_o[kMaxRows][D + 1];
  const int nthreads = blockDim.x;
#pragma unroll
  for (int h = 0; h < G; ++h) {
    if (li == 0) {
      sm_ml[rid][0] = m[h];
      sm_ml[rid][1] = l[h];
    }
#pragma unroll
    for (int e = 0; e < EPL; ++e) sm_o[rid][e0 + e] = acc[h][e];
    __syncthreads();
    for (int idx = tid; idx < a.hw * D; idx += nthreads) {
      const int hh = idx / D, d = idx - hh * D;
      float M = -INFINITY;
      for (int s2 = 0; s2 < S; ++s2) M = fmaxf(M, sm_ml[hh + s2 * a.hw][0]);
      float L = 0.f, O = 0.f;
      for (int s2 = 0; s2 < S; ++s2) {
        const int r = hh + s2 * a.hw;
        const float w = fast_exp2(sm_ml[r][0] - M);
        L = fmaf(w, sm_ml[r][1], L);
        O = fmaf(w, sm_o[r][d], O);
      }
      const size_t pidx = (size_t)((hg * a.hw + hh) * G + h) * a.n_slots + slot;
      a.ws_o[pidx * D + d] = O;
      if (d == 0) {
        a.ws_ml[pidx * 2 + 0] = M;
        a.ws_ml[pidx * 2 + 1] = L;
      }
    }
    __syncthreads();
  }
}

// Pass 1: grid (n_wg, kv-head groups). Workgroup w owns the flat token
// range [w*chunk, (w+1)*chunk) of the sequences laid end to end, so every
// workgroup but the last has the same number of tokens however ragged the
// lengths are, and the busy workgroups are the first ones dispatched. The
// range is cut at sequence boundaries into pieces; the piece of sequence b
// in workgroup w gets partial slot w + b (unique: along the stream, each
// boundary of either kind moves w or b on by at least one).
template <typename TC, int D, int G, int TPG, bool PAGED, bool PF>
__global__ __launch_bounds__(256) void k_decode_partial(DecodeArgs a) {
  const int w = blockIdx.x, hg = blockIdx.y;
  int b, off;
  locate(a, (long long)w * a.chunk, w == 0 && hg == 0, &b, &off);
  if (b < 0) return;  // uniform over the workgroup
  int budget = a.chunk;
  while (true) {
    const int n = min(clamped_len(a, b) - off, budget);
    decode_piece<TC, D, G, TPG, PAGED, PF>(a, hg, b, off, off + n, w + b);
    budget -= n;
    if (budget == 0) break;
    do {
      ++b;
    } while (b < a.B && clamped_len(a, b) == 0);
    if (b >= a.B) break;
    off = 0;
  }
}

// Online merge of pieces st, st + NS, st + 2 NS, ... of one stream, loading
// the partials of U pieces per memory round trip (k_decode_merge).
template <int U, int NS, int D, int EPL>
__device__ __forceinline__ void merge_pieces(const float* __restrict__ ws_o,
                                             const float* __restrict__ ws_ml, size_t base,
                                             int np, int st, int li, float& M, float& L,
                                             float (&O)[EPL]) {
  for (int n0 = st; n0 < np; n0 += U * NS) {
    float mn[U], ln[U], on[U][EPL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t pn = base + min(n0 + u * NS, np - 1);
      const float2 ml = *reinterpret_cast<const float2*>(ws_ml + pn * 2);
      mn[u] = ml.x;
      ln[u] = ml.y;
      const float* src = ws_o + pn * D + li * EPL;
      if constexpr (EPL == 4) {
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

// Pass 2: grid (Hq, B), 256 threads = 8 piece streams x 32 lanes; lane i of a
// stream owns elements [i*D/32, (i+1)*D/32). Sequence b's pieces are the
// slots w + b for the workgroups w its token range [cum[b], cum[b+1])
// overlaps. Each stream merges pieces n = stream, stream + 8, ... online;
// the 8 streams merge in LDS.
template <int D>
__global__ __launch_bounds__(256) void k_decode_merge(void* __restrict__ out, int out_dt,
                                                      const long long* __restrict__ cum,
                                                      const float* __restrict__ ws_o,
                                                      const float* __restrict__ ws_ml, int Hq,
                                                      int chunk, int n_wg, int n_slots,
                                                      int32_t* __restrict__ lens_inc, int cap) {
  constexpr int NS = 8;
  constexpr int EPL = D / 32;
  const int hq = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  // fused append: the sequence's length moves past its new token once pass 1
  // (which read it) has finished; nothing below reads lens
  if (lens_inc && hq == 0 && tid == 0) {
    const int p = lens_inc[b];
    if (p >= 0 && p < cap) lens_inc[b] = p + 1;
  }
  const int st = tid >> 5, li = tid & 31;
  const size_t obase = ((size_t)b * Hq + hq) * D;
  const long long c0 = cum[b], c1 = cum[b + 1];
  if (c1 <= c0) {
    if (tid < D) store_elem(out, obase + tid, out_dt, 0.f);
    return;
  }
  if (c1 > (long long)n_wg * chunk) {  // plan too small for these lengths: flag, never read past it
    if (tid < D) store_elem(out, obase + tid, out_dt, __builtin_nanf(""));
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
  if (np > 2 * NS) merge_pieces<8, NS, D, EPL>(ws_o, ws_ml, base, np, st, li, M, L, O);
  else merge_pieces<2, NS, D, EPL>(ws_o, ws_ml, base, np, st, li, M, L, O);
  __shared__ float sm_ml[NS][2];
  __shared__ float sm_o[NS][D];
  if (li == 0) {
    sm_ml[st][0] = M;
    sm_ml[st][1] = L;
  }
#pragma unroll
  for (int e = 0; e < EPL; ++e) sm_o[st][li * EPL + e] = O[e];
  __syncthreads();
  if (tid < D) {
    float MM = -INFINITY;
#pragma unroll
    for (int s = 0; s < NS; ++s) MM = fmaxf(MM, sm_ml[s][0]);
    float LL = 0.f, OO = 0.f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const float w = fast_exp2(sm_ml[s][0] - MM);  // streams with no piece: w = 0
      LL = fmaf(w, sm_ml[s][1], LL);
      OO = fmaf(w, sm_o[s][tid], OO);
    }
    store_elem(out, obase + tid, out_dt, OO / LL);
  }
}

// Kv heads per workgroup: the largest divisor of H_kv that is <= 16.
int heads_per_group(int Hkv) {
  for (int hw = kMaxRows; hw > 1; --hw)
    if (Hkv % hw == 0) return hw;
  return 1;
}

template <typename TC, int D, int G, bool PAGED>
void launch_partial(const DecodeArgs& a, hipStream_t s) {
  // Tokens per row per iteration: 8 x 16 B (or 8 x 8 B for bf16 D=64) in
  // flight per lane for K and as many for V; 4 x 32 B for fp32 D=128; and
  // 4 x 16 B for bf16 D=128 without GQA, which the plan runs at one
  // workgroup per CU on long streams: C4 158.8 -> 155.5 us per call on
  // MI355X (8 tokens in flight: 82.9% of 8 TB/s, 4: 84.6%).
  constexpr bool kMhaBf16 = sizeof(TC) == 2 && D == 128 && G == 1;
  constexpr int TPG = ((sizeof(TC) == 4 && D == 128) || kMhaBf16) ? 4 : 8;
  // Load prefetch across token groups (a second register set) for fp32
  // caches without GQA: C2/C3 measured 2-3 % faster per call on MI355X; the
  // bf16 C4 case measured 1 % slower (occupancy 4 -> 2), so it keeps one set.
  constexpr bool PF = G == 1 && sizeof(TC) == 4;
  dim3 grid(a.n_wg, a.Hkv / a.hw);
  hipLaunchKernelGGL((k_decode_partial<TC, D, G, TPG, PAGED, PF>), grid, dim3(16 * a.hw * a.S), 0,
                     s, a);
}

template <typename TC, bool PAGED>
int dispatch_partial(const DecodeArgs& a, int D, int G, hipStream_t s) {
#define SKV_DEC(DD, GG)                                    \
  if (D == DD && G == GG) {                                \
    launch_partial<TC, DD, GG, PAGED>(a, s);               \
    return 0;                                              \
  }
  SKV_DEC(64, 1) SKV_DEC(64, 2) SKV_DEC(64, 4) SKV_DEC(64, 8)
  SKV_DEC(128, 1) SKV_DEC(128, 2) SKV_DEC(128, 4) SKV_DEC(128, 8)
#undef SKV_DEC
  return set_error(SKV_E_UNSUPPORTED, "skv_decode_attn: no kernel for D=%d G=%d", D, G);
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
                  const void* new_k = nullptr, const void* new_v = nullptr, int in_dt = 0) {
  const bool app = new_k != nullptr;
  const char* fn = app ? (PAGED ? "skv_append_decode_attn_paged" : "skv_append_decode_attn")
                       : (PAGED ? "skv_decode_attn_paged" : "skv_decode_attn");
  SKV_REQUIRE(!app || (new_v && dt_ok(in_dt)), SKV_E_INVALID,
              "%s: new_v missing or bad input dtype", fn);
  SKV_REQUIRE(out && q && k && v && lens && ws, SKV_E_INVALID, "%s: null pointer argument", fn);
  SKV_REQUIRE(!PAGED || bt, SKV_E_INVALID, "%s: null block table", fn);
  SKV_REQUIRE(B > 0 && Hq > 0 && Hkv > 0, SKV_E_INVALID, "%s: dims must be > 0", fn);
  SKV_REQUIRE(B <= 65535, SKV_E_UNSUPPORTED, "%s: B=%d exceeds the grid limit", fn, B);
  SKV_REQUIRE(PAGED || T_cap > 0, SKV_E_INVALID, "%s: T_cap must be > 0", fn);
  SKV_REQUIRE(Hq % Hkv == 0, SKV_E_INVALID, "%s: H_q=%d not a multiple of H_kv=%d", fn, Hq, Hkv);
  SKV_REQUIRE(D == 64 || D == 128, SKV_E_UNSUPPORTED, "%s: D=%d (supported: 64, 128)", fn, D);
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
  a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.T_cap = T_cap;
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
  const size_t parts = (size_t)Hq * a.n_slots;
  a.ws_o = static_cast<float*>(ws);
  a.ws_ml = a.ws_o + parts * D;
  a.cum = reinterpret_cast<long long*>(a.ws_ml + parts * 2);
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
  if (D == 64)
    hipLaunchKernelGGL(k_decode_merge<64>, dim3(Hq, B), dim3(256), 0, s, out, out_dt, a.cum,
                       a.ws_o, a.ws_ml, Hq, chunk, a.n_wg, a.n_slots, lens_inc, a.cap);
  else
    hipLaunchKernelGGL(k_decode_merge<128>, dim3(Hq, B), dim3(256), 0, s, out, out_dt, a.cum,
                       a.ws_o, a.ws_ml, Hq, chunk, a.n_wg, a.n_slots, lens_inc, a.cap);
  return check_launch(fn);
}

}  // namespace
}  // namespace skv

using namespace skv;

extern "C" int skv_decode_plan(int B, int H_q, int H_kv, int max_len, long long total_len,
                               int chunk_hint, int* chunk_tokens, int* n_chunks_max) {
  SKV_REQUIRE(chunk_tokens && n_chunks_max, SKV_E_INVALID, "skv_decode_plan: null output");
  SKV_REQUIRE(B > 0 && H_q > 0 && H_kv > 0 && max_len > 0, SKV_E_INVALID,
              "skv_decode_plan: dims must be > 0 (B=%d H_q=%d H_kv=%d max_len=%d)", B, H_q, H_kv,
              max_len);
  SKV_REQUIRE(H_q % H_kv == 0, SKV_E_INVALID,
              "skv_decode_plan: H_q=%d is not a multiple of H_kv=%d", H_q, H_kv);
  int chunk;
  if (chunk_hint > 0) {
    chunk = (int)(((long)chunk_hint + 15) / 16 * 16);
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
    // 89.5% of 8 TB/s). With G = 4 (C5) the per-wavefront exp and dot work
    // needs the second workgroup: 119 -> 159 us per call at one per CU.
    const long long tot = total_len > 0 ? total_len : (long long)B * max_len;
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
  const size_t parts = (size_t)B * H_q * n_chunks_max;
  // partials (o[D], m, l) per (query head, slot), then B + 1 int64 prefix sums
  return parts * (size_t)(D + 2) * sizeof(float) + (size_t)(B + 1) * sizeof(long long);
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
