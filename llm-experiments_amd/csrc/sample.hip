// Next-token sampling on the device: repetition penalty, temperature,
// softmax, min-p, top-k and top-p filters, then one draw.
//
// Reference behaviour: sample_token (simple-llm/src/jax_backend.py:413-515),
// called by generate_text (simple-llm/src/generate.py:29-69) with the last
// repetition_window tokens of the sequence:
//   1. each distinct recent token's logit is divided by repetition_penalty
//      (a set: a token seen twice is divided once), :463-467
//   2. temperature == 0: greedy argmax (first index on ties), :470-472
//   3. p = softmax(logits / temperature), :474-477
//   4. min_p > 0: p < min_p * max(p) -> 0, renormalise, :480-486
//   5. top_k > 0: keep the top_k entries of argsort(p) (ascending, stable: of
//      equal probabilities the larger index ranks higher), renormalise, :489-495
//   6. top_p < 1: in the descending order (the reverse of that argsort),
//      keep the prefix whose running sum stays <= top_p, and always the
//      first entry; renormalise, :498-511
//   7. draw from p, :514
// The reference draws with jax.random.choice from its threefry key stream.
// Here the uniform u comes from splitmix64 (S. Vigna's public-domain mixer)
// of (seed, row, position), and the token is the first index, in index
// order, at which the running sum of p exceeds u * sum(p). So a step replayed
// from a HIP graph draws the same token.
//
// Design: one workgroup per row. Thread t holds the contiguous vocabulary
// slice [t*E, (t+1)*E) in registers (1024 x 16 or 512 x 128 entries, so
// V <= 65536),
// which makes index order the thread order for the draw and for ties. The
// top-k and top-p cut points come from a radix select over the bits of p
// (non-negative floats order like their bit patterns), 8 bits per level:
// integer counts per digit for top-k, and probability mass per digit in 2^-40
// fixed point for top-p (integer LDS atomics: exact in any order).
// Every reduction runs in a fixed order (butterfly within a wavefront, then
// the 16 wavefronts in order), so a call is bitwise reproducible.
#include "skv_common.h"

namespace skv {
namespace {

constexpr int kSampMaxWaves = 16;    // up to 1024 threads per workgroup
constexpr int kSampMaxV = 65536;     // 1024 threads x 64 or 512 threads x 128 entries

struct SampArgs {
  int32_t* out;
  float* probs_out;  // optional [M][V]: the filtered, normalised distribution
  const float* logits;
  const int32_t* seq;
  int seq_stride;
  const int32_t* lens;
  int M, V;
  float temperature;
  int top_k;
  float top_p;
  float min_p;
  float penalty;
  int window;
  unsigned long long seed;
};

// ---- fixed-order reductions over the workgroup ----------------------------

__device__ __forceinline__ float wave_sumf(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ int wave_sumi(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ float wave_maxf(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// sh: one float per wavefront of scratch. Every thread gets the result.
__device__ float block_sumf(float v, float* sh) {
  v = wave_sumf(v);
  __syncthreads();  // earlier readers of sh are done
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = 0.f;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) s += sh[w];
  return s;
}
__device__ float block_maxf(float v, float* sh) {
  v = wave_maxf(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = -INFINITY;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) s = fmaxf(s, sh[w]);
  return s;
}

// Exclusive prefix over threads in thread order; *total gets the sum.
template <typename T>
__device__ T block_excl_scan(T v, T* sh, T* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  T x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const T y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  __syncthreads();
  if (lane == 63) sh[w] = x;
  __syncthreads();
  T before = 0, all = 0;
  for (int w2 = 0; w2 < (int)(blockDim.x >> 6); ++w2) {
    if (w2 < w) before += sh[w2];
    all += sh[w2];
  }
  *total = all;
  return before + x - v;
}

constexpr int kBins = 256;            // radix digit of 8 bits: 4 levels cover the 32 bits
constexpr double kFix = 1099511627776.0;  // 2^40: fixed-point scale of probabilities

__device__ __forceinline__ long long to_fix(float p) { return (long long)((double)p * kFix); }

// The same value from the float's bits with integer shifts, for the per-entry
// path (p in [0, 1]: p * 2^40 = mantissa24 * 2^(exponent - 150 + 40)). It
// truncates like the double-based conversion for these inputs.
__device__ __forceinline__ unsigned long long to_fix_bits(uint32_t b) {
  const int e = (int)(b >> 23) & 255;
  if (e == 0) return 0ull;  // zero (and denormals, far below 2^-40)
  const unsigned long long mant = (b & 0x7FFFFFu) | 0x800000u;
  const int sh = e - 110;
  return sh >= 0 ? mant << sh : (sh > -32 ? mant >> -sh : 0ull);
}

// Walk the bins from the highest digit down, wavefront 0 only: lane l holds
// digits 4l..4l+3. Returns (through LDS) the first digit at which the running
// total (from `base`) crosses the limit -- count >= limit (top-k) or mass >
// limit (top-p) -- and the total above it; digit -1 if nothing crosses.
template <bool SUM>
__device__ void radix_walk(const int* hcnt, const long long* hsum, long long base, long long limit,
                           int* s_digit, long long* s_above) {
  const int t = threadIdx.x;
  if (t == 0) *s_digit = -1;
  if (t < 64) {
    long long c[4], own = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      c[q] = SUM ? hsum[4 * t + q] : (long long)hcnt[4 * t + q];
      own += c[q];
    }
    // total of the lanes above (higher digits)
    long long x = own;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const long long y = __shfl_down(x, o, 64);
      if (t + o < 64) x += y;
    }
    long long run = base + x - own;  // mass/count of digits above this lane's
#pragma unroll
    for (int q = 3; q >= 0; --q) {
      const bool cross = SUM ? (run + c[q] > limit) : (run + c[q] >= limit);
      if (cross) {
        if (!(SUM ? (run > limit) : (run >= limit))) {  // first crossing lies here
          *s_digit = 4 * t + q;
          *s_above = run;
        }
        break;
      }
      run += c[q];
    }
  }
  __syncthreads();
}

__device__ __forceinline__ float splitmix_uniform(unsigned long long seed, int row, int pos) {
  unsigned long long z =
      seed ^ (((unsigned long long)(unsigned)row << 32) | (unsigned long long)(unsigned)pos);
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return (float)(z >> 40) * (1.f / 16777216.f);  // 24 bits: [0, 1)
}

// Row storage of one thread: ER entries in registers and EL in LDS. Entry
// (column c, thread t) is vocabulary index c * NT + t, so every column is a
// coalesced, contiguous stretch of the row; register columns come first.
// Register entries are v[c]; LDS entry c = ER + k lives at vl[k * NT + t]
// (consecutive lanes, consecutive words).
#define SKV_EACH(BODY)                                                      \
  _Pragma("unroll") for (int c_ = 0; c_ < ER; ++c_) {                       \
    float& x = v[c_];                                                       \
    const int c = c_;                                                       \
    const int i = c_ * NT + t;                                              \
    BODY                                                                    \
  }                                                                         \
  _Pragma("unroll 4") for (int k_ = 0; k_ < EL; ++k_) {                     \
    float& x = vl[k_ * NT + t];                                             \
    const int c = ER + k_;                                                  \
    const int i = (ER + k_) * NT + t;                                       \
    BODY                                                                    \
  }

template <int ER, int EL, int NT>
__global__ __launch_bounds__(NT) void k_sample(SampArgs a) {
  constexpr int E = ER + EL;  // columns, <= 64
  static_assert(E <= 64, "column masks are 64-bit");
  __shared__ float vl[EL > 0 ? EL * NT : 1];
  // One 8 KB region serves three phases in turn (barriers in between): the
  // penalty's token bitmap, the radix bins, and the draw's per-wavefront
  // column sums.
  __shared__ __align__(16) uint32_t phase_lds[kSampMaxV / 32];
  static_assert(kBins * (sizeof(int) + sizeof(long long)) <= sizeof(phase_lds) &&
                    kSampMaxWaves * E * sizeof(float) <= sizeof(phase_lds),
                "phase region too small");
  uint32_t* mark = phase_lds;
  int* hcnt = reinterpret_cast<int*>(phase_lds);
  long long* hsum = reinterpret_cast<long long*>(phase_lds + kBins);
  float* colw = reinterpret_cast<float*>(phase_lds);  // per-wavefront column sums
  __shared__ float colsum[E];
  __shared__ int colcnt[E];
  __shared__ float shf[kSampMaxWaves];
  __shared__ int shi[kSampMaxWaves];
  __shared__ int s_digit, s_tok;
  __shared__ long long s_above;
  const int m = blockIdx.x, t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int V = a.V;
  const float* row = a.logits + (size_t)m * V;

  // Loads from clamped indices, then a select (a load under a condition
  // becomes a branch per entry and the values spill).
  float v[ER > 0 ? ER : 1];
  SKV_EACH({
    const float y = row[min(i, V - 1)];
    x = i < V ? y : -INFINITY;
  })

  // 1. repetition penalty over the set of the last `window` tokens
  const int L = min(max(a.lens[m], 0), a.seq_stride);
  if (a.penalty != 1.f && a.window > 0) {
    for (int q = t; q < (V + 31) / 32; q += NT) mark[q] = 0u;
    __syncthreads();
    for (int p = max(0, L - a.window) + t; p < L; p += NT) {
      const int tok = a.seq[(size_t)m * a.seq_stride + p];
      if (tok >= 0 && tok < V) atomicOr(&mark[tok >> 5], 1u << (tok & 31));
    }
    __syncthreads();
    SKV_EACH({
      const int ic = min(i, V - 1);
      const bool hit = i < V && ((mark[ic >> 5] >> (ic & 31)) & 1u);
      x = hit ? x / a.penalty : x;
    })
  }

  // 2. greedy: first index of the maximum
  if (a.temperature == 0.f) {
    float best = -INFINITY;
    int bi = 0x7fffffff;
    SKV_EACH({
      if (i < V && (bi == 0x7fffffff || x > best)) {  // columns ascend: first index wins
        best = x;
        bi = i;
      }
    })
    const float mx = block_maxf(best, shf);
    int cand = (best == mx) ? bi : 0x7fffffff;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) cand = min(cand, __shfl_xor(cand, o));
    __syncthreads();
    if (lane == 0) shi[w] = cand;
    __syncthreads();
    int tok = 0x7fffffff;
    for (int q = 0; q < NT / 64; ++q) tok = min(tok, shi[q]);
    if (tok == 0x7fffffff) tok = 0;
    if (t == 0) a.out[m] = tok;
    if (a.probs_out) {
      float* po = a.probs_out + (size_t)m * V;
      SKV_EACH({
        if (i < V) po[i] = i == tok ? 1.f : 0.f;
      })
    }
    return;
  }

  // 3. softmax(logits / temperature)
  float lmax = -INFINITY;
  SKV_EACH({
    x = x / a.temperature;
    lmax = fmaxf(lmax, x);
  })
  lmax = block_maxf(lmax, shf);
  float ps = 0.f;
  SKV_EACH({
    x = i < V ? expf(x - lmax) : 0.f;
    ps += x;
  })
  float Z = block_sumf(ps, shf);
  SKV_EACH({ x = x / Z; })

  // 4. min-p
  if (a.min_p > 0.f) {
    float pm = 0.f;
    SKV_EACH({ pm = fmaxf(pm, x); })
    const float thr = a.min_p * block_maxf(pm, shf);
    ps = 0.f;
    SKV_EACH({
      if (x < thr) x = 0.f;
      ps += x;
    })
    Z = block_sumf(ps, shf);
    SKV_EACH({ x = x / Z; })
  }

  // Keeps, among the entries whose bits equal TAU, the N_KEEP with the
  // largest indices (first in the descending order) and zeroes the rest:
  // columns from the top down, and inside the one column the cut straddles,
  // threads from the top down. (A macro, not a lambda: a lambda capturing the
  // register array by reference would force it into scratch memory.)
#define SKV_KEEP_TOP_TIES(TAU, N_KEEP)                                           \
  {                                                                              \
    const uint32_t tau_ = (TAU);                                                 \
    const int n_keep_ = (N_KEEP);                                                \
    if (t < E) colcnt[t] = 0;                                                    \
    __syncthreads();                                                             \
    SKV_EACH({                                                                   \
      if (i < V && __float_as_uint(x) == tau_) atomicAdd(&colcnt[c], 1);        \
    })                                                                           \
    __syncthreads();                                                             \
    int above_ = 0, cut_col_ = -1, cut_above_ = 0;                               \
    for (int q = E - 1; q >= 0; --q) {                                           \
      const int n_ = colcnt[q];                                                  \
      if (cut_col_ < 0 && above_ < n_keep_ && above_ + n_ > n_keep_) {           \
        cut_col_ = q;                                                            \
        cut_above_ = above_;                                                     \
      }                                                                          \
      above_ += n_;                                                              \
    }                                                                            \
    int rank_in_col_ = 0; /* ties of the cut column at larger threads */         \
    if (cut_col_ >= 0) {                                                         \
      int mine_ = 0;                                                             \
      SKV_EACH({                                                                 \
        if (c == cut_col_ && i < V && __float_as_uint(x) == tau_) mine_ = 1;     \
      })                                                                         \
      int tot_;                                                                  \
      const int before_ = block_excl_scan<int>(mine_, shi, &tot_);               \
      rank_in_col_ = tot_ - before_ - mine_;                                     \
    }                                                                            \
    SKV_EACH({                                                                   \
      if (i < V && __float_as_uint(x) == tau_) {                                 \
        int above_c_ = 0; /* ties in higher columns */                           \
        for (int q = c + 1; q < E; ++q) above_c_ += colcnt[q];                   \
        const bool keep_ = c == cut_col_ ? cut_above_ + rank_in_col_ < n_keep_   \
                                         : above_c_ + colcnt[c] <= n_keep_;      \
        if (!keep_) x = 0.f;                                                     \
      }                                                                          \
    })                                                                           \
  }

  // 5. top-k: tau = the k-th largest p; ties at tau keep the largest indices.
  // Zeros (dropped by min-p) are not counted: they can only be "kept" when
  // fewer than k entries are nonzero, and then every nonzero entry stays.
  // (Counted, they would all hit digit 0 of the first level at once.)
  if (a.top_k > 0 && a.top_k < V) {
    const int k = a.top_k;
    uint32_t prefix = 0;
    int above = 0;  // entries with a key above the current prefix range
    bool cut = true;
#pragma unroll 1
    for (int sh = 24; sh >= 0; sh -= 8) {
      if (t < kBins) hcnt[t] = 0;
      __syncthreads();
      const uint32_t hmask = sh >= 24 ? 0u : (0xFFFFFFFFu << (sh + 8));
      SKV_EACH({
        const uint32_t b = __float_as_uint(x);
        if (i < V && b != 0u && (b & hmask) == prefix)
          atomicAdd(&hcnt[(b >> sh) & (kBins - 1)], 1);
      })
      __syncthreads();
      radix_walk<false>(hcnt, hsum, above, k, &s_digit, &s_above);
      if (s_digit < 0) {  // fewer than k nonzero entries: nothing to cut
        cut = false;
        break;
      }
      prefix |= (uint32_t)s_digit << sh;
      above = (int)s_above;
    }
    if (cut) {
      const uint32_t tau = prefix;
      SKV_EACH({
        if (__float_as_uint(x) < tau) x = 0.f;
      })
      SKV_KEEP_TOP_TIES(tau, k - above);
    }
    ps = 0.f;
    SKV_EACH({ ps += x; })
    Z = block_sumf(ps, shf);
    SKV_EACH({ x = x / Z; })
  }

  // 6. top-p: the longest prefix of the descending order with sum <= top_p
  if (a.top_p < 1.f) {
    const long long Bfx = to_fix(a.top_p);
    uint32_t prefix = 0;
    long long acc = 0;  // mass strictly above the current prefix range
    bool all_fit = false;
#pragma unroll 1
    for (int sh = 24; sh >= 0; sh -= 8) {
      if (t < kBins) hsum[t] = 0;
      __syncthreads();
      const uint32_t hmask = sh >= 24 ? 0u : (0xFFFFFFFFu << (sh + 8));
      SKV_EACH({
        const uint32_t b = __float_as_uint(x);
        if (i < V && b != 0u && (b & hmask) == prefix)  // zeros carry no mass
          atomicAdd((unsigned long long*)&hsum[(b >> sh) & (kBins - 1)], to_fix_bits(b));
      })
      __syncthreads();
      radix_walk<true>(hcnt, hsum, acc, Bfx, &s_digit, &s_above);
      if (s_digit < 0) {  // the whole prefix range fits: keep it all, drop below
        all_fit = true;
        break;
      }
      prefix |= (uint32_t)s_digit << sh;
      acc = s_above;
    }
    if (all_fit) {
      SKV_EACH({
        if (__float_as_uint(x) < prefix) x = 0.f;
      })
    } else {
      const uint32_t tau = prefix;
      int ties = 0;
      SKV_EACH({ ties += (i < V && __float_as_uint(x) == tau) ? 1 : 0; })
      int all_ties;
      (void)block_excl_scan<int>(ties, shi, &all_ties);
      int n_fit = all_ties;
      const long long tfx = (long long)to_fix_bits(tau);
      if (tfx > 0) {
        const long long room = Bfx >= acc ? (Bfx - acc) / tfx : 0;
        n_fit = room >= all_ties ? all_ties : (int)room;
      }
      if (acc == 0 && n_fit == 0) n_fit = 1;  // the first entry always stays
      SKV_EACH({
        if (__float_as_uint(x) < tau) x = 0.f;
      })
      SKV_KEEP_TOP_TIES(tau, n_fit);
    }
    ps = 0.f;
    SKV_EACH({ ps += x; })
    Z = block_sumf(ps, shf);
    SKV_EACH({ x = x / Z; })
  }

  // 7. draw: first index whose running sum (index order) exceeds u * total.
  // Column totals first (fixed order), then the thread inside the column.
  {
    __syncthreads();
    SKV_EACH({
      const float ws = wave_sumf(x);
      if (lane == 0) colw[w * E + c] = ws;
    })
    __syncthreads();
    if (t < E) {
      float s2 = 0.f;
      for (int q = 0; q < NT / 64; ++q) s2 += colw[q * E + t];
      colsum[t] = s2;
    }
    __syncthreads();
  }
  float total = 0.f;
  for (int q = 0; q < E; ++q) total += colsum[q];
  const float target = splitmix_uniform(a.seed, m, L) * total;
  int col = -1;
  float col_base = 0.f;
  {
    float run = 0.f;
    for (int q = 0; q < E; ++q) {
      if (col < 0 && run + colsum[q] > target) {
        col = q;
        col_base = run;
      }
      run += colsum[q];
    }
  }
  if (t == 0) s_tok = -1;
  if (col >= 0) {
    float mine = 0.f;
    SKV_EACH({
      if (c == col) mine = x;
    })
    float csum;
    const float before = col_base + block_excl_scan<float>(mine, shf, &csum);
    if (mine > 0.f && before <= target && target < before + mine) s_tok = col * NT + t;
  }
  __syncthreads();
  int tok = s_tok;
  if (tok < 0) {  // rounding put the target at the very end: last nonzero entry
    int last = -1;
    SKV_EACH({
      if (i < V && x > 0.f) last = max(last, i);
    })
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) last = max(last, __shfl_xor(last, o));
    __syncthreads();
    if (lane == 0) shi[w] = last;
    __syncthreads();
    for (int q = 0; q < NT / 64; ++q) tok = max(tok, shi[q]);
    if (tok < 0) tok = 0;
  }
  if (t == 0) a.out[m] = tok;
  if (a.probs_out) {
    float* po = a.probs_out + (size_t)m * V;
    SKV_EACH({
      if (i < V) po[i] = x;
    })
  }
}
#undef SKV_KEEP_TOP_TIES
#undef SKV_EACH

// ---- split rows: unfiltered draws from wide rows ----------------------------
// Without the min-p, top-k and top-p filters (the reference's defaults,
// generate.py:8-18) a draw needs only each row's softmax sum and one pass
// over the stretch where the running sum crosses u * sum. A row of 8192 or
// more entries is cut into slices of kSliceV entries, one workgroup each:
// k_sample_slices writes the slice's max and its sum of exp(x - max) (after
// the penalty and the temperature, fixed order); then k_sample_pick, one
// workgroup per row, weighs the slices by exp(max - row max) in slice order,
// finds the slice where the running sum crosses u * sum, recomputes that
// slice's entries alone and takes the first index, in index order, whose
// running sum exceeds the target: the rule of k_sample, with the sums
// grouped by slice (a draw within float rounding of a step of the running
// sum may differ from k_sample's). A row of 50,304 entries is then 25
// workgroups reading 8 KB each instead of one reading 200 KB at one CU's rate.
constexpr int kSliceThreads = 256;
constexpr int kSliceEPT = 8;                         // entries per thread
constexpr int kSliceV = kSliceThreads * kSliceEPT;  // 2048
constexpr int kSplitMinV = 8192;
constexpr int kMaxSlices = kSampMaxV / kSliceV;     // 32

// Penalty marks of the slice [lo, lo + kSliceV) of row m: bit j of mark is
// set when token lo + j (< V) is among the row's last `window` tokens.
__device__ void slice_marks(const SampArgs& a, int m, int L, int lo, uint32_t* mark) {
  const int t = threadIdx.x;
  if (t < kSliceV / 32) mark[t] = 0u;
  __syncthreads();
  for (int p = max(0, L - a.window) + t; p < L; p += kSliceThreads) {
    const int tok = a.seq[(size_t)m * a.seq_stride + p];
    const int j = tok - lo;
    if (tok >= 0 && tok < a.V && j >= 0 && j < kSliceV) atomicOr(&mark[j >> 5], 1u << (j & 31));
  }
  __syncthreads();
}

// Grid (S, M): stats[m][s] = (max, sum of exp(x - max)) of slice s of row m,
// x = logit (/ penalty) / temperature; a slice with no finite entry gives
// (-inf, 0). Thread t holds entries lo + j * 256 + t (coalesced loads).
__global__ __launch_bounds__(kSliceThreads) void k_sample_slices(SampArgs a,
                                                                 float2* __restrict__ stats,
                                                                 int S) {
  __shared__ uint32_t mark[kSliceV / 32];
  __shared__ float sh[kSliceThreads / 64];
  const int s = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
  const int V = a.V, lo = s * kSliceV;
  const float* row = a.logits + (size_t)m * V;
  float x[kSliceEPT];
#pragma unroll
  for (int j = 0; j < kSliceEPT; ++j) {
    const int i = lo + j * kSliceThreads + t;
    const float y = row[min(i, V - 1)];
    x[j] = i < V ? y : -INFINITY;
  }
  if (a.penalty != 1.f && a.window > 0) {
    slice_marks(a, m, min(max(a.lens[m], 0), a.seq_stride), lo, mark);
#pragma unroll
    for (int j = 0; j < kSliceEPT; ++j) {
      const int k = j * kSliceThreads + t;
      if ((mark[k >> 5] >> (k & 31)) & 1u) x[j] = x[j] / a.penalty;
    }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < kSliceEPT; ++j) {
    x[j] = x[j] / a.temperature;
    mx = fmaxf(mx, x[j]);
  }
  mx = block_maxf(mx, sh);
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < kSliceEPT; ++j) sum += x[j] == -INFINITY ? 0.f : expf(x[j] - mx);
  sum = block_sumf(sum, sh);
  if (t == 0) stats[(size_t)m * S + s] = make_float2(mx, sum);
}

// Grid (M): the draw of row m from the slice statistics (see above). Thread
// t of the picked slice holds its entries lo + 8 t .. lo + 8 t + 7 (index
// order within the thread, then across threads).
__global__ __launch_bounds__(kSliceThreads) void k_sample_pick(SampArgs a,
                                                               const float2* __restrict__ stats,
                                                               int S) {
  __shared__ uint32_t mark[kSliceV / 32];
  __shared__ float sh[kSliceThreads / 64];
  __shared__ float s_w[kMaxSlices], s_mx[kMaxSlices];
  __shared__ int s_i[kSliceThreads / 64];
  const int m = blockIdx.x, t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int V = a.V;
  const int L = min(max(a.lens[m], 0), a.seq_stride);
  const float2 st = t < S ? stats[(size_t)m * S + t] : make_float2(-INFINITY, 0.f);
  const float rmax = block_maxf(st.x, sh);
  if (t < S) {
    s_mx[t] = st.x;
    // a slice without mass weighs 0 (also when no slice has any: rmax = -inf);
    // a NaN sum stays NaN
    s_w[t] = st.y == 0.f ? 0.f : st.y * expf(st.x - rmax);
  }
  __syncthreads();
  float total = 0.f;
  for (int q = 0; q < S; ++q) total += s_w[q];
  const float target = splitmix_uniform(a.seed, m, L) * total;
  int sel = -1;
  float base = 0.f;
  {
    float run = 0.f;
    for (int q = 0; q < S; ++q) {
      if (sel < 0 && run + s_w[q] > target) {
        sel = q;
        base = run;
      }
      run += s_w[q];
    }
    if (sel < 0 && total == total) {  // rounding put the target at the very end
      for (int q = 0; q < S; ++q)
        if (s_w[q] > 0.f) {
          sel = q;
          base = run - s_w[q];  // not exact: only the last entry can then match
        }
    }
  }
  int tok = 0;  // no mass, or a NaN anywhere in the row: token 0, as k_sample
  if (sel >= 0) {  // uniform
    const int lo = sel * kSliceV;
    const float* row = a.logits + (size_t)m * V;
    const bool pen = a.penalty != 1.f && a.window > 0;
    if (pen) slice_marks(a, m, L, lo, mark);
    const float smx = s_mx[sel], scale = expf(smx - rmax);
    float p[kSliceEPT];
    float mine = 0.f;
#pragma unroll
    for (int j = 0; j < kSliceEPT; ++j) {
      const int k = kSliceEPT * t + j, i = lo + k;
      float x = row[min(i, V - 1)];
      if (pen && ((mark[k >> 5] >> (k & 31)) & 1u)) x = x / a.penalty;
      x = x / a.temperature;
      p[j] = (i < V && x != -INFINITY) ? expf(x - smx) * scale : 0.f;
      mine += p[j];
    }
    float all;
    float r = base + block_excl_scan<float>(mine, sh, &all);
    int found = 0x7fffffff, last = -1;
#pragma unroll
    for (int j = 0; j < kSliceEPT; ++j) {
      const int i = lo + kSliceEPT * t + j;
      if (p[j] > 0.f) {
        if (found == 0x7fffffff && r <= target && target < r + p[j]) found = i;
        last = i;
      }
      r += p[j];
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      found = min(found, __shfl_xor(found, o));
      last = max(last, __shfl_xor(last, o));
    }
    __syncthreads();
    if (lane == 0) s_i[w] = found;
    __syncthreads();
    int f = 0x7fffffff;
    for (int q = 0; q < kSliceThreads / 64; ++q) f = min(f, s_i[q]);
    __syncthreads();
    if (lane == 0) s_i[w] = last;
    __syncthreads();
    int lst = -1;
    for (int q = 0; q < kSliceThreads / 64; ++q) lst = max(lst, s_i[q]);
    // no crossing inside the slice (its recomputed sum fell short of the
    // target by rounding): its last entry with mass
    tok = f != 0x7fffffff ? f : (lst >= 0 ? lst : 0);
  }
  if (t == 0) a.out[m] = tok;
}

// Slices of a row for the split path, 0 when the row takes k_sample.
int sample_slices(int V) {
  return V >= kSplitMinV && V <= kSampMaxV ? (V + kSliceV - 1) / kSliceV : 0;
}

}  // namespace
}  // namespace skv

using namespace skv;

extern "C" size_t skv_sample_workspace_bytes(int M, int V) {
  const int S = sample_slices(V);
  return M > 0 && S > 0 ? (size_t)M * S * sizeof(float2) : 0;
}

extern "C" int skv_sample(int32_t* out, float* probs_out, const float* logits, const int32_t* seq,
                          int seq_stride, const int32_t* lens, int M, int V, float temperature,
                          int top_k, float top_p, float min_p, float repetition_penalty,
                          int repetition_window, unsigned long long seed, void* ws,
                          size_t ws_bytes, skv_stream_t stream) {
  const char* fn = "skv_sample";
  SKV_REQUIRE(out && logits && seq && lens, SKV_E_INVALID, "%s: null pointer argument", fn);
  SKV_REQUIRE(M > 0 && V > 0 && seq_stride > 0, SKV_E_INVALID, "%s: dims must be > 0", fn);
  SKV_REQUIRE(M <= 65535, SKV_E_UNSUPPORTED, "%s: M=%d exceeds the grid limit", fn, M);
  SKV_REQUIRE(V <= kSampMaxV, SKV_E_UNSUPPORTED, "%s: V=%d > %d", fn, V, kSampMaxV);
  SKV_REQUIRE(temperature >= 0.f, SKV_E_INVALID, "%s: temperature must be >= 0", fn);
  SKV_REQUIRE(top_k >= 0 && min_p >= 0.f && repetition_penalty > 0.f && repetition_window >= 0,
              SKV_E_INVALID, "%s: bad filter parameters", fn);
  SampArgs a{out, probs_out, logits, seq, seq_stride, lens, M, V, temperature, top_k, top_p,
             min_p, repetition_penalty, repetition_window, seed};
  hipStream_t s = (hipStream_t)stream;
  // Unfiltered draws from wide rows: the split path, given the workspace.
  const int S = sample_slices(V);
  if (temperature > 0.f && top_k == 0 && top_p >= 1.f && min_p == 0.f && probs_out == nullptr &&
      S > 0 && ws != nullptr && ws_bytes >= skv_sample_workspace_bytes(M, V)) {
    float2* stats = static_cast<float2*>(ws);
    hipLaunchKernelGGL(k_sample_slices, dim3(S, M), dim3(kSliceThreads), 0, s, a, stats, S);
    hipLaunchKernelGGL(k_sample_pick, dim3(M), dim3(kSliceThreads), 0, s, a, stats, S);
    return check_launch(fn);
  }
  // 1024 threads; entries per thread in registers (ER) and in LDS (EL):
  // 16 register columns fit without spilling, so rows up to 53248 entries
  // (GPT-2's 50304) keep 36 more columns in LDS; rows up to 65536 take 28
  // register columns and spill a little.
  const int per = (V + 1023) / 1024;
  if (per <= 4)
    hipLaunchKernelGGL((k_sample<4, 0, 1024>), dim3(M), dim3(1024), 0, s, a);
  else if (per <= 16)
    hipLaunchKernelGGL((k_sample<16, 0, 1024>), dim3(M), dim3(1024), 0, s, a);
  else if (per <= 52)
    hipLaunchKernelGGL((k_sample<16, 36, 1024>), dim3(M), dim3(1024), 0, s, a);
  else
    hipLaunchKernelGGL((k_sample<28, 36, 1024>), dim3(M), dim3(1024), 0, s, a);
  return check_launch(fn);
}
