// Cached single-query decode attention: split-K (flash-decoding) kernels on
// gfx950, shared by the head-dim-specific translation units
// (decode_attn.hip: D = 64 and 128; decode_attn_generic.hip: any other D).
//
// Reference behaviour: attention_with_kv_cache
// (simple-llm/src/gpu/gpu_kv_cache.py:194-289) launches
// create_attention_with_kv_cache_kernel (simple-llm/src/gpu/gpu_kernels.py:2801-2938):
// per (b, h), s_t = scale * q . K[t] for t < len, softmax over [0, len),
// o = sum_t p_t V[t]. One workgroup per (b, h), len <= 256, and any head_dim
// (the kernel loops over head_dim, :2856-2866 and :2916-2921).
//
// Design (HBM-bound GEMV, no MFMA):
//  * Pass 1, grid (workgroup, kv-head group). The sequences' filled tokens,
//    laid end to end, form one flat stream; workgroup w owns its tokens
//    [w*chunk, (w+1)*chunk), cut into pieces at sequence boundaries, for a
//    group of HW kv heads. Equal ranges keep a ragged batch as evenly spread
//    over the CUs as a uniform one. A workgroup is made of 16-lane DPP rows:
//    row r serves kv head r % HW of the group and token substream r / HW
//    (S substreams, HW*S <= 16). Lane i of a row owns elements
//    [i*DP/16, (i+1)*DP/16) of each K and V row it reads, DP being the head
//    dim padded to a power of two (32..256): lanes past the real head dim
//    D read an in-row address, meet a zero query and store nothing. Loads
//    are vectors (16 bytes at D = 64/128, the widest that divides D
//    otherwise). Because the cache is [B, T, H_kv, D], the HW heads of one
//    token are contiguous: a wavefront (4 rows) reads 4 consecutive head
//    rows of the same token (1 KB for bf16 D=128), and the workgroup sweeps
//    whole token rows in address order. This keeps HBM reads contiguous;
//    reading one head's 256-byte rows at a 4 KB stride measured ~11% slower
//    on MI355X. The loads are non-temporal.
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
#pragma once

#include "skv_common.h"

namespace skv {
namespace dec {

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
  int D;         // head dim (the row stride of q, out, caches and partials)
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

// Pass 1 of a head dim other than 64 and 128: launches the masked
// k_decode_partial for D <= 256, G in {1, 2, 4, 8} (G = 8 needs D <= 128).
// Returns 0, or an SKV_E_UNSUPPORTED status. Contiguous caches:
// decode_attn_generic.hip; paged: decode_attn_generic_paged.hip.
int launch_partial_generic(const DecodeArgs& a, int G, bool bf16_cache, hipStream_t s);
int launch_partial_generic_paged(const DecodeArgs& a, int G, bool bf16_cache, hipStream_t s);

// Pass 1 on the matrix cores for grouped queries (decode_gqa_mfma.hip):
// bf16 caches, head dim 64 or 128, G in {2, 4, 8}, pages of >= 16 tokens or
// a contiguous capacity that is a multiple of 16.
bool gqa_mfma_eligible(const DecodeArgs& a, int G, bool bf16_cache, bool paged);
int launch_partial_gqa(const DecodeArgs& a, int G, bool paged, hipStream_t s);

// Largest head dim the masked kernels take with G query heads per kv head:
// G * head_dim <= 4096 and head_dim <= 2048 (wavefront rows of up to 32
// elements a lane).
inline int max_head_dim(int G) { return G <= 2 ? 2048 : 4096 / G; }

// Kv heads per workgroup: the largest divisor of H_kv that is <= 16.
inline int heads_per_group(int Hkv) {
  for (int hw = kMaxRows; hw > 1; --hw)
    if (Hkv % hw == 0) return hw;
  return 1;
}

}  // namespace dec

namespace {

using dec::DecodeArgs;
using dec::kMaxRows;

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

// Row of kv head hk at position t of sequence b; rows are RS elements apart.
template <typename TC, bool PAGED>
__device__ __forceinline__ const TC* row_ptr(const TC* base, const DecodeArgs& a, int b, int t,
                                             int hk, int RS) {
  size_t row;
  if constexpr (PAGED) {
    const int blk = a.block_table[(size_t)b * a.max_blocks + (t >> a.bs_shift)];
    row = ((size_t)blk << a.bs_shift) + (t & ((1 << a.bs_shift) - 1));
  } else {
    row = (size_t)b * a.T_cap + t;
  }
  return base + (row * a.Hkv + hk) * RS;
}

// A lane's fragment of one K/V row for a head dim below the padded DP (or
// without a 16-byte vector that divides it): EPL = DP/16 elements read as
// EPL/VG groups of VG elements (VG divides D, so a group lies wholly inside
// or wholly past the row). eo[j] is group j's element offset in the row: its
// own for a group inside, 0 for one past D (an in-row address whose values
// meet a zero query and feed an accumulator slot that is never stored).
template <typename TC, int EPL, int VG>
struct FragM {
  static constexpr int NG = EPL / VG;
  static constexpr int GBYTES = VG * (int)sizeof(TC);
  static constexpr bool PACK = sizeof(TC) == 2 && VG >= 2;  // two bf16 per word
  static constexpr int NW = PACK ? EPL / 2 : EPL;
  static constexpr int WPG = NW / NG;  // words per group
  uint32_t w[NW];
  __device__ __forceinline__ void load(const TC* row, const int (&eo)[NG]) {
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const TC* p = row + eo[j];
      if constexpr (GBYTES == 16) {
        const u32x4_t x = stream_load16(p);
        w[j * 4 + 0] = x.x; w[j * 4 + 1] = x.y; w[j * 4 + 2] = x.z; w[j * 4 + 3] = x.w;
      } else if constexpr (GBYTES == 8) {
        const u32x2_t x = stream_load8(p);
        w[j * 2 + 0] = x.x; w[j * 2 + 1] = x.y;
      } else if constexpr (GBYTES == 4) {
        w[j] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
      } else {  // one bf16: kept in the high half, so the word is its fp32 value
        static_assert(GBYTES == 2, "group size");
        w[j] = (uint32_t)__builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(p)) << 16;
      }
    }
  }
  __device__ __forceinline__ float get(int e) const {
    if constexpr (PACK) return (e & 1) ? bf16w_hi(w[e >> 1]) : bf16w_lo(w[e >> 1]);
    else return __uint_as_float(w[e]);
  }
};

// Fragment type of a row: the exact-D form (Frag, whole 8- or 16-byte
// vectors) or the masked one.
template <typename TC, int EPL, int VG, bool MASK>
struct FragSel {
  using type = Frag<TC, EPL>;
};
template <typename TC, int EPL, int VG>
struct FragSel<TC, EPL, VG, true> {
  using type = FragM<TC, EPL, VG>;
};

// Position `first` of the flat token stream (the sequences' filled tokens
// laid end to end) -> (sequence, offset in it), or sequence -1 past the end.
// Rounds of blockDim sequences: an inclusive scan of the clamped lengths
// within each wavefront (shuffles, no barrier), then across the wavefronts
// through LDS. The workgroup with write_cum also stores the exclusive prefix
// sums (and the total at [B]) for the merge pass.
__device__ void locate(const DecodeArgs& a, long long first, bool write_cum, int* b_out,
                       int* off_out) {
  __shared__ long long s_wave[16];  // wavefront totals of one round (blockDim <= 1024)
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

// Sum over the LANES lanes of a row: 16 (one DPP row) or 64 (a whole
// wavefront: the DPP row sums, then across the four rows).
template <int LANES>
__device__ __forceinline__ float lanes_sum(float x) {
  x = row16_sum(x);
  if constexpr (LANES == 64) {
    x += __shfl_xor(x, 16);
    x += __shfl_xor(x, 32);
  }
  return x;
}

// Tokens [start, end) of sequence b for the workgroup's kv heads -> one
// partial per query head at `slot`. D is the padded head dim (the real one,
// a.D, when !MASK); VG the elements per load of the masked form. LANES: the
// lanes of a row, 16 (a DPP row) or 64 (a wavefront, for head dims whose
// query and accumulators do not fit 16 lanes' registers).
template <typename TC, int D, int G, int TPG, bool PAGED, bool PF, int VG, bool MASK,
          int LANES = 16>
__device__ __forceinline__ void decode_piece(const DecodeArgs& a, int hg, int b, int start,
                                             int end, int slot) {
  static_assert(!(PF && MASK), "the prefetching loop takes exact head dims");
  static_assert(LANES == 16 || LANES == 64, "a row is a DPP row or a wavefront");
  constexpr int EPL = D / LANES;
  constexpr int ROWS = 256 / LANES;  // rows of a full workgroup
  using FragT = typename FragSel<TC, EPL, VG, MASK>::type;
  constexpr int NG = EPL / VG;
  const int RS = MASK ? a.D : D;  // row stride of q, caches and partials
  const int tid = threadIdx.x;
  const int rid = tid / LANES;  // row
  const int li = tid % LANES;   // lane within the row
  const int e0 = li * EPL;
  const int hl = rid % a.hw;  // kv head within the group
  const int sub = rid / a.hw; // token substream
  const int hk = hg * a.hw + hl;
  const int S = a.S;
  // masked form: element e of this lane is inside the row iff e0 + e < RS
  int eo[NG];
#pragma unroll
  for (int j = 0; j < NG; ++j) eo[j] = (!MASK || e0 + j * VG < RS) ? e0 + j * VG : 0;
  auto inside = [&](int e) { return !MASK || e0 + e < RS; };

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
    const size_t qoff = ((size_t)b * a.Hq + hk * G + h) * RS + e0;
    if constexpr (MASK) {
      // element loads at clamped offsets; lanes past D get a zero query
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float v = load_elem(a.q, inside(e) ? qoff + e : 0, a.q_dt);
        q[h][e] = inside(e) ? v * a.qscale : 0.f;
      }
    } else if constexpr (PF) {
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
#define SKV_FRAG_LOAD_(F, P)                                                  \
  {                                                                           \
    if constexpr (MASK) F.load(P, eo);                                        \
    else F.load((P) + e0);                                                    \
  }
#define SKV_LOAD_TILE_(KF, VF, T0, FLOOR)                                     \
  {                                                                           \
    _Pragma("unroll") for (int u = 0; u < TPG; ++u) {                         \
      int t_ = min((T0) + u, mend - 1);                                        \
      if (FLOOR) t_ = max(t_, 0);                                             \
      SKV_FRAG_LOAD_(KF[u], (row_ptr<TC, PAGED>(kb, a, b, t_, hk, RS)));      \
    }                                                                         \
    _Pragma("unroll") for (int u = 0; u < TPG; ++u) {                         \
      int t_ = min((T0) + u, mend - 1);                                        \
      if (FLOOR) t_ = max(t_, 0);                                             \
      SKV_FRAG_LOAD_(VF[u], (row_ptr<TC, PAGED>(vb, a, b, t_, hk, RS)));      \
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
        d = lanes_sum<LANES>(d);                                              \
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
    FragT ka[TPG], va[TPG], kn[TPG], vn[TPG];
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
      FragT kf[TPG], vf[TPG];
      SKV_LOAD_TILE(kf, vf, t0);
      SKV_CONSUME(kf, vf, t0);
    }
  }
#undef SKV_CONSUME
#undef SKV_LOAD_TILE
#undef SKV_LOAD_TILE_
#undef SKV_FRAG_LOAD_

  if (has_new && sub == 0) {
    // The appended token: the input row, rounded to the cache's precision,
    // is stored at position end - 1 and attended like the cached ones.
    const int tn = end - 1;
    float kx[EPL], vx[EPL];
    const size_t src = ((size_t)b * a.Hkv + hk) * RS + e0;
    TC* kdst = const_cast<TC*>(row_ptr<TC, PAGED>(kb, a, b, tn, hk, RS)) + e0;
    TC* vdst = const_cast<TC*>(row_ptr<TC, PAGED>(vb, a, b, tn, hk, RS)) + e0;
    if constexpr (MASK) {
      // element loads at clamped offsets, element stores inside the row only
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        kx[e] = load_elem(a.new_k, inside(e) ? src + e : 0, a.in_dt);
        vx[e] = load_elem(a.new_v, inside(e) ? src + e : 0, a.in_dt);
        if constexpr (sizeof(TC) == 2) {  // attended as stored: rounded to bf16
          kx[e] = bf16_to_f32(f32_to_bf16(kx[e]));
          vx[e] = bf16_to_f32(f32_to_bf16(vx[e]));
        }
      }
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        if (!inside(e)) continue;
        if constexpr (sizeof(TC) == 2) {
          kdst[e] = f32_to_bf16(kx[e]);  // exact: kx[e] is bf16 already
          vdst[e] = f32_to_bf16(vx[e]);
        } else {
          kdst[e] = kx[e];
          vdst[e] = vx[e];
        }
      }
    } else {
      if constexpr (EPL == 8) {
        load8_f32(a.new_k, src, a.in_dt, kx);
        load8_f32(a.new_v, src, a.in_dt, vx);
      } else {
        load4_f32(a.new_k, src, a.in_dt, kx);
        load4_f32(a.new_v, src, a.in_dt, vx);
      }
      store_row<TC, EPL>(kdst, kx);
      store_row<TC, EPL>(vdst, vx);
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) d = fmaf(q[h][e], kx[e], d);
      d = lanes_sum<LANES>(d);
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
      for (int e = 0; e < EPL; ++e)
        if (inside(e)) a.ws_o[pidx * RS + e0 + e] = acc[h][e];
      if (li == 0) {
        a.ws_ml[pidx * 2 + 0] = m[h];
        a.ws_ml[pidx * 2 + 1] = l[h];
      }
    }
    return;
  }

  // S > 1: merge the S substreams of each head through LDS, one query head
  // at a time. Rows that saw no token drop out through exp2(-inf) = 0.
  __shared__ float sm_ml[ROWS][2];
  __shared__ float sm_o[ROWS][D + 1];
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
    for (int idx = tid; idx < a.hw * RS; idx += nthreads) {
      const int hh = idx / RS, d = idx - hh * RS;
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
      a.ws_o[pidx * RS + d] = O;
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
template <typename TC, int D, int G, int TPG, bool PAGED, bool PF, int VG, bool MASK,
          int LANES = 16>
__global__ __launch_bounds__(256) void k_decode_partial(DecodeArgs a) {
  const int w = blockIdx.x, hg = blockIdx.y;
  int b, off;
  locate(a, (long long)w * a.chunk, w == 0 && hg == 0, &b, &off);
  if (b < 0) return;  // uniform over the workgroup
  int budget = a.chunk;
  while (true) {
    const int n = min(clamped_len(a, b) - off, budget);
    decode_piece<TC, D, G, TPG, PAGED, PF, VG, MASK, LANES>(a, hg, b, off, off + n, w + b);
    budget -= n;
    if (budget == 0) break;
    do {
      ++b;
    } while (b < a.B && clamped_len(a, b) == 0);
    if (b >= a.B) break;
    off = 0;
  }
}

template <typename TC, int D, int G, int TPG, bool PAGED, bool PF, int VG, bool MASK,
          int LANES = 16>
void launch_partial_t(const DecodeArgs& a, hipStream_t s) {
  dim3 grid(a.n_wg, a.Hkv / a.hw);
  hipLaunchKernelGGL((k_decode_partial<TC, D, G, TPG, PAGED, PF, VG, MASK, LANES>), grid,
                     dim3(LANES * a.hw * a.S), 0, s, a);
}

// ---------------------------------------------------------------------------
// Head dims other than 64 and 128: the head dim padded to DP, a power of two
// in [32, 256]; lane i of a 16-lane row owns elements [i*DP/16,
// (i+1)*DP/16), and lanes (or parts of a lane) past the real head dim read
// an in-row address, meet a zero query and store nothing. Loads are the
// widest vector that divides D (up to 16 bytes), or single elements.
// ---------------------------------------------------------------------------

// Tokens in flight per row and iteration, from a register budget: the
// query and accumulator of G heads take 2*G*EPL registers, each K and V
// fragment NW words.
template <typename TC, int DP, int G, int VG, int LANES>
constexpr int tokens_per_group() {
  constexpr int EPL = DP / LANES;
  constexpr int NW = (sizeof(TC) == 2 && VG >= 2) ? EPL / 2 : EPL;
  constexpr int budget = 160 - 2 * G * EPL;
  constexpr int t = budget / (2 * NW);
  return t >= 8 ? 8 : t >= 4 ? 4 : t >= 2 ? 2 : 1;
}

// Whether G query heads of a DP-wide head fit a lane's registers with rows
// of LANES lanes: the queries and accumulators take 2*G*DP/LANES of them.
template <int DP, int G, int LANES>
constexpr bool fits() {
  return 2 * G * (DP / LANES) <= 128;
}

template <typename TC, int DP, int G, int VG, bool PAGED, int LANES>
int launch_g(const DecodeArgs& a, hipStream_t s) {
  if constexpr (!fits<DP, G, LANES>()) {
    return set_error(SKV_E_UNSUPPORTED,
                     "skv_decode_attn: no kernel for head_dim %d with %d query heads per kv head "
                     "(G * head_dim up to 4096)",
                     a.D, G);
  } else if constexpr (LANES == 16) {
    launch_partial_t<TC, DP, G, tokens_per_group<TC, DP, G, VG, 16>(), PAGED, false, VG, true>(
        a, s);
    return 0;
  } else {
    // Rows are wavefronts: a workgroup of 4 serves up to 4 kv heads (the
    // largest divisor of H_kv that is <= 4), the rest of its rows split the
    // tokens of each head into substreams.
    DecodeArgs w = a;
    w.hw = 1;
    for (int hw = 4; hw > 1; --hw)
      if (a.Hkv % hw == 0) {
        w.hw = hw;
        break;
      }
    w.S = 4 / w.hw;
    launch_partial_t<TC, DP, G, tokens_per_group<TC, DP, G, VG, 64>(), PAGED, false, VG, true,
                     64>(w, s);
    return 0;
  }
}

template <typename TC, int DP, bool PAGED, int LANES>
int launch_dp(const DecodeArgs& a, int G, hipStream_t s) {
  constexpr int EPL = DP / LANES;
  constexpr int WIDE = sizeof(TC) == 4 ? (EPL < 4 ? EPL : 4) : (EPL < 8 ? EPL : 8);
  const bool wide = a.D % WIDE == 0;
#define SKV_G(GG)                                                               \
  if (G == GG)                                                                  \
    return wide ? launch_g<TC, DP, GG, WIDE, PAGED, LANES>(a, s)                \
                : launch_g<TC, DP, GG, 1, PAGED, LANES>(a, s);
  SKV_G(1) SKV_G(2) SKV_G(4) SKV_G(8)
#undef SKV_G
  return set_error(SKV_E_UNSUPPORTED, "skv_decode_attn: no kernel for G=%d", G);
}

// The masked pass 1 for this head dim, cache dtype and layout: rows of 16
// lanes up to a padded head dim of 256 (128 with G = 8), wavefront rows past
// that, up to max_head_dim(G).
template <typename TC, bool PAGED>
int launch_generic(const DecodeArgs& a, int G, hipStream_t s) {
  if (a.D < 1 || a.D > dec::max_head_dim(G))
    return set_error(SKV_E_UNSUPPORTED,
                     "skv_decode_attn: head_dim %d with %d query heads per kv head (supported: "
                     "1 to %d)",
                     a.D, G, dec::max_head_dim(G));
  if (a.D <= 32) return launch_dp<TC, 32, PAGED, 16>(a, G, s);
  if (a.D <= 64) return launch_dp<TC, 64, PAGED, 16>(a, G, s);
  if (a.D <= 128) return launch_dp<TC, 128, PAGED, 16>(a, G, s);
  if (a.D <= 256 && G < 8) return launch_dp<TC, 256, PAGED, 16>(a, G, s);
  if (a.D <= 256) return launch_dp<TC, 256, PAGED, 64>(a, G, s);
  if (a.D <= 512) return launch_dp<TC, 512, PAGED, 64>(a, G, s);
  if (a.D <= 1024) return launch_dp<TC, 1024, PAGED, 64>(a, G, s);
  return launch_dp<TC, 2048, PAGED, 64>(a, G, s);
}

}  // namespace
}  // namespace skv
