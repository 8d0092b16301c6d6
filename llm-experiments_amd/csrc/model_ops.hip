// Decode-step ops of the model around the KV-cache path (fp32).
//
// Reference model (simple-llm/src/jax_backend.py):
//   x = embedding[ids] + pos_encoding[pos]                       :144
//   layer_norm(x) = (x - mean) / sqrt(var + 1e-5) * g + b         :78-82
//   q, k, v = x . Wq, x . Wk, x . Wv; out = attn . Wo             :110-122
//   ff = gelu_tanh(x . W1 + b1) . W2 + b2                        :125-129
//   logits = x . embedding^T                                     :147
//   greedy token = argmax(logits), first index on ties            :466-469
// generate_text (simple-llm/src/generate.py:29-69) feeds the prompt and then
// the argmax of every step; skv_next_tokens does that choice on the device so
// a whole decode step needs no host round trip.
//
// Linear layers are skinny GEMMs (a few rows per step) bound by reading the
// weights from HBM. They run on fp32 MFMA (v_mfma_f32_16x16x4_f32): a
// workgroup owns 16 output columns and up to 64 rows; its wavefronts split
// K, each feeding one 16x16 tile per 16-row block, and the partial tiles are
// summed through LDS before the fused epilogue (bias, GELU, residual). The
// LayerNorm in front of a projection can be folded into its x reads.
// Weights are stored transposed, Wt[N][K], so every lane reads 16
// contiguous bytes of a weight row per step.
#include <type_traits>

#include "skv_common.h"

namespace skv {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// ---------------------------------------------------------------------------
// embedding + positional encoding
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_embed(float* __restrict__ x, const int32_t* __restrict__ ids,
                                               const int32_t* __restrict__ pos,
                                               const float* __restrict__ emb,
                                               const float* __restrict__ pe, int d, int vocab,
                                               int ctx) {
  const int m = blockIdx.x;
  const int id = min(max(ids[m], 0), vocab - 1);
  const int p = min(max(pos[m], 0), ctx - 1);
  for (int j = threadIdx.x; j < d; j += blockDim.x)
    x[(size_t)m * d + j] = emb[(size_t)id * d + j] + pe[(size_t)p * d + j];
}

// ---------------------------------------------------------------------------
// LayerNorm: one workgroup (256 threads) per row, two-pass mean / variance
// ---------------------------------------------------------------------------
constexpr int kLnMaxPerThread = 16;  // d <= 4096

__device__ __forceinline__ float block_sum(float v, float* sh) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) sh[w] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) t += sh[i];
  return t;
}

__global__ __launch_bounds__(256) void k_layernorm(float* __restrict__ y, const float* __restrict__ x,
                                                   const float* __restrict__ gamma,
                                                   const float* __restrict__ beta, int d,
                                                   float eps) {
  __shared__ float sh[4];
  const int m = blockIdx.x;
  const float* xr = x + (size_t)m * d;
  float v[kLnMaxPerThread];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kLnMaxPerThread; ++i) {
    const int j = threadIdx.x + i * 256;
    v[i] = j < d ? xr[j] : 0.f;
    s += v[i];
  }
  const float mean = block_sum(s, sh) / d;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < kLnMaxPerThread; ++i) {
    const int j = threadIdx.x + i * 256;
    const float c = j < d ? v[i] - mean : 0.f;
    q += c * c;
  }
  const float rstd = 1.f / sqrtf(block_sum(q, sh) / d + eps);
#pragma unroll
  for (int i = 0; i < kLnMaxPerThread; ++i) {
    const int j = threadIdx.x + i * 256;
    if (j < d) y[(size_t)m * d + j] = (v[i] - mean) * rstd * gamma[j] + beta[j];
  }
}

// ---------------------------------------------------------------------------
// Linear: y = act(x Wt^T + bias) + res, MFMA fp32
// ---------------------------------------------------------------------------
constexpr int kNumCUs = 256;          // compute units of an MI355X
constexpr int kLinRowsPerBlock = 64;  // 4 tiles of 16 rows
constexpr int kLinMaxWaves = 16;      // wavefronts per workgroup, splitting K

__device__ __forceinline__ float gelu_tanh(float v) {
  const float k0 = 0.7978845608028654f;  // sqrt(2 / pi)
  return 0.5f * v * (1.f + tanhf(k0 * (v + 0.044715f * v * v * v)));
}

// Barrier over the workgroup's LDS only: each wavefront waits for its own LDS
// operations, not for its global loads and stores (__syncthreads() waits for
// those too: before the logits' argmax step it waited for the logits' own
// stores, ~3 us a call).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// argmax step: (v, i) replaces the best (bv, bi) if v is larger, or equal
// with a smaller index (the first maximum wins; NaN never does)
__device__ __forceinline__ void better(float& bv, int& bi, float v, int i) {
  // selects, not a branch: a branch split every use into basic blocks, so
  // the loads feeding a chain of these could not be issued together
  const bool take = v > bv || (v == bv && i < bi);
  bv = take ? v : bv;
  bi = take ? i : bi;
}

struct LinArgs {
  float* y;
  const float* x;
  const float* wt;
  const float* bias;
  const float* res;
  const float* ln_g;  // optional LayerNorm of the x rows, applied on the fly
  const float* ln_b;
  float ln_eps;
  int M, N, K;
  int act;      // 0 none, 1 gelu (tanh form)
  int split;    // > 0: column n goes to segment n / split of a [N/split][M][split] output
  int kz;       // K range of one workgroup along grid z (a multiple of 16; K when unsplit)
  float* part;  // split K: raw partial sums [grid z][M][N]; the reduce pass finishes them
  float* cand;  // k_linear_wide: per-row argmax candidates [M][grid] values, then indices
};

// Lane layout of v_mfma_f32_16x16x4_f32: operand A lane l holds
// (m = l % 16, k = l / 16), operand B holds (k = l / 16, n = l % 16), and
// result slot i holds (m = 4 * (l / 16) + i, n = l % 16). Within each step
// of 16 k the four MFMAs take k = k0 + 4 * (l / 16) + i for i = 0..3 from
// the same 16-byte load of x and of Wt (a consistent permutation of k).
//
// The W wavefronts of a workgroup (W = blockDim / 64) split K in contiguous
// ranges of STEPS 16-wide steps and sum their tiles through LDS; no
// workgroup waits on another. Each wavefront issues every load it needs --
// its weights, its x values, gamma and beta, and for the epilogue threads the
// bias and residual -- before it uses any of them, so a projection costs one
// HBM round trip for the weights, overlapped with the LayerNorm statistics,
// instead of one per unrolled round: at these sizes (M <= 64 rows, a few MB
// of weights) a CU's weight stream is latency-bound, so the number of
// dependent round trips sets the time. K beyond W * STEPS * 16 (K > 3072 for
// 16 wavefronts of 12 steps) runs in further passes.
//
// With LN, each x row is layer-normalized as it is read: the mean and 1/std
// of the workgroup's rows are computed first (sums of the values shifted by
// the row's first element, var = E[(x-c)^2] - E[x-c]^2), which takes the
// LayerNorm launch out of the step. When one pass of the workgroup covers all
// of K, its wavefronts already hold every x value of their rows, and the sums
// come from those registers (reduced across lanes and then wavefronts through
// LDS); otherwise a separate pass reads the rows again. Skipping that second
// read of x took the 16 x 768 -> 2304 projection from 9.4 to 7.4 us.
// Passes of more than 4 steps run with 8 wavefronts, which leaves each up to
// 256 registers.
template <int TILES, int STEPS, bool LN, bool SPREAD>
__global__ __launch_bounds__(STEPS > 4 ? 512 : kLinMaxWaves * 64) void k_linear(LinArgs a) {
  // 16-byte aligned: the dynamic block starts after the static variables, at
  // their size rounded up to this alignment, and is read as float4
  extern __shared__ __attribute__((aligned(16))) float red[];  // partial tiles of the W wavefronts
  __shared__ float stat[kLinRowsPerBlock][2];
  // Row statistics from the registers when a pass covers all of K, for one
  // row tile and passes of 4+ steps: with fewer, the x rows are short (the
  // second read costs little) and the cross-wavefront sum of 16 wavefronts
  // costs more (16 x 256 -> 768: 0.25 us slower, measured on MI355X).
  constexpr bool kRegStats = LN && TILES == 1 && STEPS >= 4;
  __shared__ float lsum[kRegStats ? kLinMaxWaves : 1][16][2];
  const int NW = blockDim.x >> 6;
  const int n0 = blockIdx.x * 16;
  const int m0 = blockIdx.y * kLinRowsPerBlock;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int lr = l & 15, lk = l >> 4;
  const int rows = min(TILES * 16, a.M - m0);
  const int n = n0 + lr;
  const bool n_ok = n < a.N;
  const float* wrow = a.wt + (size_t)(n_ok ? n : 0) * a.K;
  // Loads read a clamped, in-bounds address and select zero afterwards: a
  // load inside a condition cannot be hoisted, and the compiler then splits
  // it into four guarded 4-byte loads. K % 4 == 0, so K - 4 starts a float4.
  // The selects come after the scheduling barrier below, so that no use of a
  // loaded value sits among the loads: with one there, the scheduler may wait
  // for each load before issuing the next to save registers (seen at 6 steps:
  // 12 round trips in series).
  const int klast = a.K - 4;
  auto load4 = [](const float* p) { return *reinterpret_cast<const float4*>(p); };
  auto keep = [](float4& v, bool ok) {
    if (!ok) v = make_float4(0.f, 0.f, 0.f, 0.f);
  };

  // Epilogue: thread (wave, l) finishes accumulator slots p (j = 0..3) of
  // lane l: row tile t = p / 4, slot i = p % 4, row m0 + 16 t + 4 (l / 16) + i,
  // column nn. SPREAD (the host sets it for M > 4) spreads the slots over
  // all wavefronts (p = wave + j NW; partials lane-contiguous in LDS,
  // [W][TILES][4][64]). Otherwise (M <= 4: the valid slots are row tile 0's
  // first ones anyway) wavefront t < TILES takes row tile t (p = 4 wave + j;
  // partials [W][TILES][64][4], one 16-byte LDS write per lane). Measured on
  // MI355X: spreading took C3 (16 rows) from 704 to 674 us per step; the
  // compact form saved C1 (1 row) 4 us. Each kernel carries one form only (a
  // runtime choice between the two was slower for both). Bias and residual
  // values are loaded now, with everything else.
  constexpr bool spread = SPREAD;
  const bool partial = a.part != nullptr;  // split K: raw sums, no epilogue here
  const int nn = n0 + (l & 15);
  const bool n_in = nn < a.N;
  auto slot_of = [&](int j) { return spread ? wave + j * NW : 4 * wave + j; };
  auto slot_row = [&](int p) { return m0 + 16 * (p >> 2) + 4 * (l >> 4) + (p & 3); };
  float bias_v = 0.f, resv[4] = {0.f, 0.f, 0.f, 0.f};
  size_t oidx[4] = {0, 0, 0, 0};
  if (n_in && !partial && (spread || wave < TILES)) {
    if (a.bias) bias_v = a.bias[nn];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int p = slot_of(j), m = slot_row(p);
      if (p >= 4 * TILES || m >= a.M) continue;
      if (a.split > 0) {
        const int seg = nn / a.split;
        oidx[j] = ((size_t)seg * a.M + m) * a.split + (nn - seg * a.split);
      } else {
        oidx[j] = (size_t)m * a.N + nn;
      }
      if (a.res) resv[j] = a.res[oidx[j]];
    }
  }

  f32x4 acc[TILES];
#pragma unroll
  for (int t = 0; t < TILES; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int pass_k = NW * STEPS * 16;
  const int kz0 = blockIdx.z * a.kz;
  const int kz1 = min(a.K, kz0 + a.kz);
  // LN statistics from the registers (one row tile): one pass holds all of K
  const bool whole = kRegStats && kz0 == 0 && kz1 == a.K && pass_k >= a.K;
  const float cshift = kRegStats ? a.x[(size_t)(m0 + min(lr, rows - 1)) * a.K] : 0.f;
  for (int kp = kz0; kp < kz1; kp += pass_k) {
    const int kb = kp + wave * STEPS * 16 + 4 * lk;
    float4 w[STEPS], xv[TILES][STEPS], g[LN ? STEPS : 1], be[LN ? STEPS : 1];
#pragma unroll
    for (int st = 0; st < STEPS; ++st) w[st] = load4(wrow + min(kb + 16 * st, klast));
#pragma unroll
    for (int t = 0; t < TILES; ++t)
#pragma unroll
      for (int st = 0; st < STEPS; ++st)
        xv[t][st] = load4(a.x + (size_t)(m0 + min(t * 16 + lr, rows - 1)) * a.K +
                          min(kb + 16 * st, klast));
    if constexpr (LN) {
#pragma unroll
      for (int st = 0; st < STEPS; ++st) {
        g[st] = load4(a.ln_g + min(kb + 16 * st, klast));
        be[st] = load4(a.ln_b + min(kb + 16 * st, klast));
      }
    }
    // keep every load above issued before the first use below
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int st = 0; st < STEPS; ++st) {
      const bool kin = kb + 16 * st < kz1;
      keep(w[st], n_ok && kin);
#pragma unroll
      for (int t = 0; t < TILES; ++t) keep(xv[t][st], t * 16 + lr < rows && kin);
      if constexpr (LN) {
        keep(g[st], kin);
        keep(be[st], kin);
      }
    }
    if constexpr (LN) {
      if (kp == kz0 && whole) {
        // lanes lr + 16 j (j = 0..3) of every wavefront hold row lr
        float su = 0.f, sq = 0.f;
#pragma unroll
        for (int st = 0; st < STEPS; ++st) {
          if (kb + 16 * st >= kz1) continue;
          const float4 v = xv[0][st];
          const float d0 = v.x - cshift, d1 = v.y - cshift, d2 = v.z - cshift, d3 = v.w - cshift;
          su += (d0 + d1) + (d2 + d3);
          sq += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
        }
        su += __shfl_xor(su, 16);
        sq += __shfl_xor(sq, 16);
        su += __shfl_xor(su, 32);
        sq += __shfl_xor(sq, 32);
        if (lk == 0) {
          lsum[wave][lr][0] = su;
          lsum[wave][lr][1] = sq;
        }
        __syncthreads();
        if (wave == 0 && lk == 0) {
          su = 0.f;
          sq = 0.f;
          for (int wv = 0; wv < NW; ++wv) {
            su += lsum[wv][lr][0];
            sq += lsum[wv][lr][1];
          }
          const float ms = su / a.K;
          stat[lr][0] = cshift + ms;
          stat[lr][1] = 1.f / sqrtf(fmaxf(sq / a.K - ms * ms, 0.f) + a.ln_eps);
        }
        __syncthreads();
      } else if (kp == kz0) {
        // row statistics over the whole row, one wavefront per row
        for (int r = wave; r < rows; r += NW) {
          const float* xr = a.x + (size_t)(m0 + r) * a.K;
          const float c = xr[0];
          float sum = 0.f, sq = 0.f;
          for (int j = l; j < a.K; j += 64) {
            const float v = xr[j] - c;
            sum += v;
            sq += v * v;
          }
          const float ms = wave_sum(sum) / a.K;
          const float mean = c + ms;
          const float rstd = 1.f / sqrtf(fmaxf(wave_sum(sq) / a.K - ms * ms, 0.f) + a.ln_eps);
          if (l == 0) {
            stat[r][0] = mean;
            stat[r][1] = rstd;
          }
        }
        __syncthreads();
      }
#pragma unroll
      for (int t = 0; t < TILES; ++t) {
        const int r = t * 16 + lr;
        if (r >= rows) continue;  // those x values are zero already
        const float mu = stat[r][0], rs = stat[r][1];
#pragma unroll
        for (int st = 0; st < STEPS; ++st) {
          if (kb + 16 * st >= kz1) continue;
          float4& v = xv[t][st];
          v.x = (v.x - mu) * rs * g[st].x + be[st].x;
          v.y = (v.y - mu) * rs * g[st].y + be[st].y;
          v.z = (v.z - mu) * rs * g[st].z + be[st].z;
          v.w = (v.w - mu) * rs * g[st].w + be[st].w;
        }
      }
    }
#pragma unroll
    for (int st = 0; st < STEPS; ++st)
#pragma unroll
      for (int t = 0; t < TILES; ++t) {
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[t][st].x, w[st].x, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[t][st].y, w[st].y, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[t][st].z, w[st].z, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[t][st].w, w[st].w, acc[t], 0, 0, 0);
      }
  }
  auto red_at = [&](int wv, int p) -> float& {
    return spread ? red[((wv * TILES + (p >> 2)) * 4 + (p & 3)) * 64 + l]
                   : red[((wv * TILES + (p >> 2)) * 64 + l) * 4 + (p & 3)];
  };
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) red_at(wave, 4 * t + i) = acc[t][i];
  __syncthreads();
  if (!n_in || (!spread && wave >= TILES)) return;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int p = slot_of(j), m = slot_row(p);
    if (p >= 4 * TILES || m >= a.M) continue;
    float v = bias_v;  // then the wavefronts' partial sums, in order
    for (int wv = 0; wv < NW; ++wv) v += red_at(wv, p);
    if (partial) {
      a.part[((size_t)blockIdx.z * a.M + m) * a.N + nn] = v;
      continue;
    }
    if (a.act == 1) v = gelu_tanh(v);
    a.y[oidx[j]] = v + resv[j];
  }
}

// Wide projections of one row tile (M <= 16 rows, at least 1024 16-column
// tiles: the tied logits, 16 x 768 -> 50304). k_linear gives each 16-column
// tile its own workgroup, which reads the whole x block (as many bytes as
// its weights) and reduces across wavefronts; at 3,144 tiles that halved the
// useful stream of every CU (154.5 MB in ~45 us, 3.4 TB/s). Here one
// workgroup per CU stages the x rows once in LDS (LayerNorm applied there)
// and takes a contiguous range of column tiles, 12-13 for the logits. Each
// tile is cut into four K quarters; the quarter units are dealt to the 8
// wavefronts round-robin, so the CUs and the wavefronts stream equal byte
// counts, and a unit's US weight loads (16 bytes per lane each) are issued
// together. The four quarter partials of a tile are summed in LDS in a
// fixed order (bitwise reproducible), then the epilogue adds bias and
// residual and applies the activation.
//
// PACKED: the weights come in the MFMA lane order of skv_linear_pack
// (tile-major, then 16-k steps, then lane, 16 bytes a lane), so the 64 lanes
// of one step load 1 KB of consecutive bytes and a quarter unit is one
// contiguous block; in the [N, K] layout a step reads 64 bytes from each of
// 16 rows, which streamed ~8 % slower on MI355X (24.4 against 22.4 us for
// the logits' 154.5 MB, loads only).
constexpr int kWideWaves = 8;
constexpr int kWideMaxTiles = 16;  // column tiles per workgroup (N <= 65536 on 256 CUs)

template <int US, bool LN, bool PACKED = false, int NW = kWideWaves, bool CAND = false>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(NW / 4, NW / 4)))
void k_linear_wide(LinArgs a, int tiles_total) {
  static_assert(!CAND || PACKED, "argmax candidates come with the packed weights only");
  constexpr int PARTS = NW / 2;  // K parts of a tile (units), 16 US columns of K each
  // 16-byte aligned: the dynamic block starts after the static variables, at
  // their size rounded up to this alignment, and is read as float4 (after the
  // 2052 bytes of the candidates' variables it started misaligned by 4, and
  // the packed logits took 33-36 instead of 29 us)
  extern __shared__ __attribute__((aligned(16))) float wsm[];  // x rows [16][K + 4], then partials
  __shared__ float wstat[16][2];
  // argmax candidates (CAND): per-wavefront bests, arrivals
  __shared__ float s_cv[CAND ? NW : 1][16];
  __shared__ int s_ci[CAND ? NW : 1][16];
  __shared__ unsigned s_done;
  if (CAND && threadIdx.x == 0) s_done = 0;  // used after the barrier below
  const int K = a.K, P = K + 4;   // K = 16 * US * PARTS
  float* xs = wsm;
  float* part = wsm + 16 * P;
  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63, lr = l & 15, lk = l >> 4;
  const int M = a.M;
  // this workgroup's column tiles [t0, t1)
  const int G = gridDim.x;
  const int t0 = (int)((long long)blockIdx.x * tiles_total / G);
  const int t1 = (int)((long long)(blockIdx.x + 1) * tiles_total / G);
  const int nt = t1 - t0;
  // this wavefront's units: u_k = wave + NW k, k < nk (u = PARTS j + q: part
  // q of tile j)
  const int nk = (PARTS * nt - wave + NW - 1) / NW;
  auto issue = [&](int k, float4 (&w)[US]) {
    // past the last unit the wavefront re-reads its last one (an L2 hit):
    // loads behind a condition would make the compiler wait for both sets
    const int u = wave + NW * min(k, max(nk - 1, 0));
    const int j = u / PARTS, q = u % PARTS;
    if constexpr (PACKED) {
      // tile t0 + j, steps [q US, (q + 1) US): 256 floats a step, streamed
      // (non-temporal: 32.3 -> 30.8 us for the cold logits on MI355X)
      const float* wp = a.wt + (((size_t)(t0 + j) * (K / 16) + q * US) * 64 + l) * 4;
#pragma unroll
      for (int st = 0; st < US; ++st) {
        const u32x4_t t = stream_load16(wp + 256 * st);
        w[st] = make_float4(__uint_as_float(t[0]), __uint_as_float(t[1]), __uint_as_float(t[2]),
                            __uint_as_float(t[3]));
      }
    } else {
      const int n = min((t0 + j) * 16 + lr, a.N - 1);
      const float* wp = a.wt + (size_t)n * K + q * (K / PARTS) + 4 * lk;
#pragma unroll
      for (int st = 0; st < US; ++st) w[st] = *reinterpret_cast<const float4*>(wp + 16 * st);
    }
    // keep the loads here: the scheduler would otherwise move them down next
    // to their use, one unit's latency per unit
    __builtin_amdgcn_sched_barrier(0);
  };
  // x rows (16 x K, rows past M read row 0 and are zeroed): US / 2 float4
  // per thread, loaded first; then the first unit's weights, so both round
  // trips overlap (loads complete in issue order, so x can be waited for
  // while the weights are still in flight); then x goes to LDS
  constexpr int XV = US / 2;  // 16 K / 4 / (NW * 64) float4 a thread
  float4 xr[XV], gr[LN ? XV : 1], br[LN ? XV : 1];
#pragma unroll
  for (int v = 0; v < XV; ++v) {
    const int i = (tid + v * NW * 64) * 4;
    const int r = i / K, k = i - r * K;
    xr[v] = *reinterpret_cast<const float4*>(a.x + (size_t)(r < M ? r : 0) * K + k);
  }
  if constexpr (LN) {
    // the norm's scale and shift at the same positions, so that nothing
    // after this waits on a global load while the weights are in flight
#pragma unroll
    for (int v = 0; v < XV; ++v) {
      const int k = ((tid + v * NW * 64) * 4) % K;
      gr[v] = *reinterpret_cast<const float4*>(a.ln_g + k);
      br[v] = *reinterpret_cast<const float4*>(a.ln_b + k);
    }
  }
  float4 wa[US], wb[US];
  issue(0, wa);
#pragma unroll
  for (int v = 0; v < XV; ++v) {
    const int i = (tid + v * NW * 64) * 4;
    const int r = i / K, k = i - r * K;
    if (r >= M) xr[v] = make_float4(0.f, 0.f, 0.f, 0.f);
    *reinterpret_cast<float4*>(xs + r * P + k) = xr[v];
  }
  __syncthreads();
  if constexpr (LN) {
    // row statistics (sums shifted by the row's first element), 16 / NW rows
    // per wavefront, then the rows normalized in place
    for (int r = wave * (16 / NW); r < (wave + 1) * (16 / NW); ++r) {
      const float c = xs[r * P];
      float su = 0.f, sq = 0.f;
      for (int k = l; k < K; k += 64) {
        const float d = xs[r * P + k] - c;
        su += d;
        sq += d * d;
      }
      su = wave_sum(su);
      sq = wave_sum(sq);
      if (l == 0) {
        const float ms = su / K;
        wstat[r][0] = c + ms;
        wstat[r][1] = 1.f / sqrtf(fmaxf(sq / K - ms * ms, 0.f) + a.ln_eps);
      }
    }
    __syncthreads();
    // each thread normalizes the elements it staged (rows past M stay zero)
#pragma unroll
    for (int v = 0; v < XV; ++v) {
      const int i = (tid + v * NW * 64) * 4;
      const int r = i / K, k = i - r * K;
      if (r >= M) continue;
      const float mu = wstat[r][0], rs = wstat[r][1];
      float4 x = xr[v];
      x.x = (x.x - mu) * rs * gr[v].x + br[v].x;
      x.y = (x.y - mu) * rs * gr[v].y + br[v].y;
      x.z = (x.z - mu) * rs * gr[v].z + br[v].z;
      x.w = (x.w - mu) * rs * gr[v].w + br[v].w;
      *reinterpret_cast<float4*>(xs + r * P + k) = x;
    }
    __syncthreads();
  }

  // unit u_k from the weights in w
  auto compute = [&](int k, const float4 (&w)[US]) {
    const int u = wave + NW * k;
    const int q = u % PARTS;
    const float* xp = xs + lr * P + q * (K / PARTS) + 4 * lk;
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < US; ++st) {
      const float4 xv = *reinterpret_cast<const float4*>(xp + 16 * st);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.x, w[st].x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.y, w[st].y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.z, w[st].z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.w, w[st].w, acc, 0, 0, 0);
    }
    *reinterpret_cast<f32x4*>(part + ((size_t)u * 64 + l) * 4) = acc;
  };
  // two units in flight per wavefront: unit k + 1 loads while unit k is
  // consumed. The body has no branch between a load and its use (with one the
  // compiler sinks the loads next to their use and the overlap is lost); an
  // odd last unit is done after the loop.
  int k = 0;
  for (; k + 1 < nk; k += 2) {
    issue(k + 1, wb);
    compute(k, wa);
    issue(k + 2, wa);
    compute(k + 1, wb);
  }
  if (k < nk) compute(k, wa);
  lds_barrier();  // the partials; a clamped re-read may still be in flight
  // epilogue: tile j by wavefront j % NW; slot i of lane l is row 4 lk + i, column lr.
  // With CAND (a.cand given, packed weights) each row's first maximum over this workgroup's
  // columns is tracked as well: per lane, then over the 16 columns of a lane
  // group, then over the wavefronts in LDS, in an order-independent way
  // (larger value, or equal value and smaller column).
  float cbv[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  int cbi[4] = {a.N, a.N, a.N, a.N};
  for (int j = wave; j < nt; j += NW) {
    const int n = (t0 + j) * 16 + lr;
    if (n >= a.N) continue;
    f32x4 v = *reinterpret_cast<const f32x4*>(part + ((size_t)(PARTS * j) * 64 + l) * 4);
#pragma unroll
    for (int q = 1; q < PARTS; ++q)
      v += *reinterpret_cast<const f32x4*>(part + ((size_t)(PARTS * j + q) * 64 + l) * 4);
    const float bv = a.bias ? a.bias[n] : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 4 * lk + i;
      if (m >= M) continue;
      float y = v[i] + bv;
      if (a.act == 1) y = gelu_tanh(y);
      if (a.res) y += a.res[(size_t)m * a.N + n];
      a.y[(size_t)m * a.N + n] = y;
      if constexpr (CAND) better(cbv[i], cbi[i], y, n);
    }
  }
  if constexpr (CAND) {
    // Per row, the best of the 16 columns of a lane group by DPP row shifts
    // (lane 15 of the group ends with all 16); each wavefront's bests go to
    // LDS, it counts itself done on an LDS counter, and the last wavefront to
    // arrive reduces the NW of them and writes the workgroup's candidates: no
    // barrier. (Cross-lane shuffles and a barrier before a reduction by 16
    // threads cost the projection ~3 us a call; every wavefront writing its
    // own candidates, 16 times as many, slowed the picking.)
    auto shr_step = [&](auto n) {  // lane j of a row takes lane j - n's (row_shr:n)
      constexpr int ctl = 0x110 + decltype(n)::value;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float ov = __int_as_float(__builtin_amdgcn_update_dpp(
            __float_as_int(cbv[i]), __float_as_int(cbv[i]), ctl, 0xF, 0xF, false));
        const int oi = __builtin_amdgcn_update_dpp(cbi[i], cbi[i], ctl, 0xF, 0xF, false);
        better(cbv[i], cbi[i], ov, oi);
      }
    };
    shr_step(std::integral_constant<int, 1>{});
    shr_step(std::integral_constant<int, 2>{});
    shr_step(std::integral_constant<int, 4>{});
    shr_step(std::integral_constant<int, 8>{});
    if (lr == 15) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s_cv[wave][4 * lk + i] = cbv[i];
        s_ci[wave][4 * lk + i] = cbi[i];
      }
    }
    int last = 0;
    if (l == 0)
      last = __hip_atomic_fetch_add(&s_done, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP) ==
             (unsigned)(NW - 1);
    if (!__builtin_amdgcn_readfirstlane(last)) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    if (l < M) {
      float vv[NW];
      int ii[NW];
#pragma unroll
      for (int w = 0; w < NW; ++w) {  // every read issued before the first compare
        vv[w] = s_cv[w][l];
        ii[w] = s_ci[w][l];
      }
      float bv = -INFINITY;
      int bi = a.N;
#pragma unroll
      for (int w = 0; w < NW; ++w) better(bv, bi, vv[w], ii[w]);
      const int G = gridDim.x;
      a.cand[(size_t)l * G + blockIdx.x] = bv;
      reinterpret_cast<int*>(a.cand + (size_t)M * G)[(size_t)l * G + blockIdx.x] = bi;
    }
  }
}

// Skinny projections (M <= 16 rows, one row tile) with K = 16 * STEPS * NW:
// one 16-column tile per workgroup, wavefront w taking the K range
// [16 STEPS w, 16 STEPS (w + 1)). A decode step's projections are a few MB
// each (16 x 768 -> 2304 is 7.1 MB), so one HBM round trip of every
// workgroup's loads, the products and one cross-wavefront sum set the time;
// per-phase clocks on MI355X showed that what costs is what a CU returns to
// its registers (weights and x rows, 16 bytes a lane each, as many bytes of
// x as of weights) and every wait between phases. So:
//  - every load (weights, x, and the epilogue's bias, residual and
//    LayerNorm terms) is issued before the first use, weights and x
//    interleaved by step, so the products of step s start when step s has
//    arrived;
//  - with LN the weights come folded (skv_linear_fold_ln): w' = gamma * w,
//    c1[n] = sum_k w'[n, k], c2[n] = beta . w[n, :] + bias[n], and
//      LN(x) . w^T + bias = rstd (sum_k (x - c) w' - (mean - c) c1) + c2
//    for any shift c (c = x[m, 0] here, so that neither the sums of the row
//    statistics nor the products cancel against a large mean). The products
//    run on raw x as soon as it lands, the row sums of (x - c) and (x - c)^2
//    come from the same registers, and both meet in the epilogue after the
//    one barrier; gamma and beta are never loaded (16 x 768 -> 2304 with
//    LN: 8.0 -> 6.1 us a call, weights streamed from HBM, on MI355X).
// Rows past M read row M - 1 (their results are dropped), so no load is
// conditional. The NW wavefront partials are summed in order in LDS.
//
// CAND (no LN; a.cand given): the workgroup also writes each row's first
// maximum over its 16 columns (larger value, or equal value and smaller
// column; NaN never wins) to a.cand[m][blockIdx.x], values then columns, by
// DPP row shifts over the 16 epilogue lanes of the row: no LDS, no barrier.
//
// Split K (grid.y = S > 1, no LN): workgroup (j, z) takes the K range
// [z K / S, (z + 1) K / S) of tile j, for narrow layers with too few tiles
// to occupy the CUs (16 x 3072 -> 768: 48 tiles). The last of a tile's S
// workgroups to finish sums the S partial tiles, in z order, and runs the
// epilogue; no second launch. A device-scope fence in every workgroup would
// write back its XCD's L2 (~30 us a call, measured on MI355X), so the
// partials instead go out as device-scope atomic stores, which write
// through to memory: each thread waits until its store is acknowledged
// before the workgroup's barrier, one thread then counts the arrival with a
// device-scope atomic add, and the last arriver reads the partials with
// device-scope atomic loads, which are served from memory. The arrival
// counters (one per tile, in the caller's workspace) start at zero and the
// last arriver puts its tile's back to zero.
template <int STEPS, bool LN, bool CAND = false>
__global__ __launch_bounds__(1024) void k_linear_skinny(LinArgs a, const float* __restrict__ c1,
                                                        unsigned* __restrict__ cnt) {
  static_assert(!CAND || !LN, "candidates only without LayerNorm");
  // 16-byte aligned (read as float4; see k_linear_wide)
  extern __shared__ __attribute__((aligned(16))) float sred[];  // [NW][64][4] partial tiles, then [NW][16][2] row sums
  const int NW = blockDim.x >> 6;
  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63, lr = l & 15, lk = l >> 4;
  const int M = a.M, K = a.K, N = a.N;
  const int n0 = blockIdx.x * 16;
  // epilogue operands: thread t < 256 finishes y[m = t / 16, n0 + t % 16]
  const int em = tid >> 4, en = n0 + (tid & 15);
  const int emc = min(em, M - 1), enc = min(en, N - 1);
  size_t oidx = (size_t)emc * N + enc;
  if (a.split > 0) {
    const int seg = enc / a.split;
    oidx = ((size_t)seg * M + emc) * a.split + (enc - seg * a.split);
  }
  const float e_bias = a.bias ? a.bias[enc] : 0.f;
  const float e_res = a.res ? a.res[oidx] : 0.f;
  const float e_c1 = LN ? c1[enc] : 0.f;
  // this lane's x row (the A operand's row is lane % 16) and its shift
  const int rx = min(lr, M - 1);
  const float cs = LN ? a.x[(size_t)rx * K] : 0.f;
  const int kb = blockIdx.y * a.kz + wave * (STEPS * 16) + 4 * lk;
  const float* wp = a.wt + (size_t)min(n0 + lr, N - 1) * K + kb;
  const float* xp = a.x + (size_t)rx * K + kb;
  float4 w[STEPS], xv[STEPS];
#pragma unroll
  for (int st = 0; st < STEPS; ++st) {
    w[st] = *reinterpret_cast<const float4*>(wp + 16 * st);
    xv[st] = *reinterpret_cast<const float4*>(xp + 16 * st);
  }
  __builtin_amdgcn_sched_barrier(0);
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  float su = 0.f, sq = 0.f;
#pragma unroll
  for (int st = 0; st < STEPS; ++st) {
    float4 v = xv[st];
    if constexpr (LN) {
      v.x -= cs;
      v.y -= cs;
      v.z -= cs;
      v.w -= cs;
      su += (v.x + v.y) + (v.z + v.w);
      sq += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
    }
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(v.x, w[st].x, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(v.y, w[st].y, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(v.z, w[st].z, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(v.w, w[st].w, acc, 0, 0, 0);
  }
  // slot i of lane l: row 4 (l / 16) + i, column l % 16
  *reinterpret_cast<f32x4*>(sred + ((size_t)wave * 64 + l) * 4) = acc;
  float* rsum = sred + (size_t)NW * 256;
  if constexpr (LN) {
    // lanes lr, lr + 16, lr + 32, lr + 48 hold row lr
    su += __shfl_xor(su, 16);
    sq += __shfl_xor(sq, 16);
    su += __shfl_xor(su, 32);
    sq += __shfl_xor(sq, 32);
    if (lk == 0) {
      rsum[(wave * 16 + lr) * 2] = su;
      rsum[(wave * 16 + lr) * 2 + 1] = sq;
    }
  }
  __syncthreads();
  const bool et = tid < 256;
  const int pl = 16 * (em >> 2) + (en - n0), pi = em & 3;
  float v = 0.f;
  if (et)
    for (int wv = 0; wv < NW; ++wv) v += sred[((size_t)wv * 64 + pl) * 4 + pi];
  const int S = gridDim.y;
  if (!LN && S > 1) {
    __shared__ unsigned s_last;
    float* pt = a.part + (size_t)blockIdx.x * S * 256;
    if (et) __hip_atomic_store(pt + blockIdx.y * 256 + tid, v, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);  // the write-through store is acknowledged
    __syncthreads();
    if (tid == 0)
      s_last = __hip_atomic_fetch_add(cnt + blockIdx.x, 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(S - 1);
    __syncthreads();
    if (!s_last) return;
    if (tid == 0) __hip_atomic_store(cnt + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (!et) return;
    float pz[8];
    v = 0.f;
    for (int z0 = 0; z0 < S; z0 += 8) {  // up to 8 loads in flight, summed in z order
#pragma unroll
      for (int i = 0; i < 8; ++i)
        pz[i] = __hip_atomic_load(pt + min(z0 + i, S - 1) * 256 + tid, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (z0 + i < S) v += pz[i];
    }
  }
  const bool live = et && em < M && en < N;
  if (!CAND && !live) return;
  if (live) {
    if constexpr (LN) {
      float s1 = 0.f, s2 = 0.f;
      for (int wv = 0; wv < NW; ++wv) {
        s1 += rsum[(wv * 16 + em) * 2];
        s2 += rsum[(wv * 16 + em) * 2 + 1];
      }
      const float ms = s1 / K;  // mean - c
      const float rstd = 1.f / sqrtf(fmaxf(s2 / K - ms * ms, 0.f) + a.ln_eps);
      v = rstd * (v - ms * e_c1);
    }
    v += e_bias;
    if (a.act == 1) v = gelu_tanh(v);
    v += e_res;
    a.y[oidx] = v;
  }
  if constexpr (CAND) {
    if (!et || 4 * wave >= M) return;  // whole wavefronts: rows 4 wave .. 4 wave + 3
    float bv = -INFINITY;
    int bi = N;
    if (live) better(bv, bi, v, en);
    auto shr_step = [&](auto n) {  // lane j of a row takes lane j - n's (row_shr:n)
      constexpr int ctl = 0x110 + decltype(n)::value;
      const float ov = __int_as_float(
          __builtin_amdgcn_update_dpp(__float_as_int(bv), __float_as_int(bv), ctl, 0xF, 0xF, false));
      const int oi = __builtin_amdgcn_update_dpp(bi, bi, ctl, 0xF, 0xF, false);
      better(bv, bi, ov, oi);
    };
    shr_step(std::integral_constant<int, 1>{});
    shr_step(std::integral_constant<int, 2>{});
    shr_step(std::integral_constant<int, 4>{});
    shr_step(std::integral_constant<int, 8>{});
    if ((tid & 15) == 15 && em < M) {  // lane 15 of the row holds all 16
      const int G = gridDim.x;
      a.cand[(size_t)em * G + blockIdx.x] = bv;
      reinterpret_cast<int*>(a.cand + (size_t)M * G)[(size_t)em * G + blockIdx.x] = bi;
    }
  }
}

// Steps per wavefront of k_linear_skinny for this K (NW = K / (16 STEPS)
// wavefronts, 4..16), 0 when none fits. At K = 768 (and each 768-wide split
// of K = 3072) 8 wavefronts of 6 steps measured best on MI355X, weights cold:
// q/k/v 6.17 us against 6.32 (16 x 3) and 6.60 (4 x 12), MLP up 6.40 against
// 6.54 and 6.83, MLP down 7.20 against 7.36; C3 595.5 against 599.1 us per step.
int skinny_steps(int K) {
  for (int st : {6, 4, 3, 8, 12}) {
    if (K % (16 * st)) continue;
    const int nw = K / (16 * st);
    if (nw >= 4 && nw <= 16) return st;
  }
  return 0;
}

// K splits of k_linear_skinny for a projection without LayerNorm: narrow
// layers (fewer than 128 tiles) split until about 192 workgroups, keeping
// every split's K range a k_linear_skinny shape.
int skinny_splits(int M, int N, int K) {
  const int tiles = (N + 15) / 16;
  if (M > 16 || tiles >= 128) return 1;
  int best = 1;
  for (int S : {2, 3, 4, 6, 8}) {
    if (K % S || skinny_steps(K / S) == 0 || (long)tiles * S > 256) continue;
    best = S;
  }
  return best;
}

// Workspace of the M <= 64 paths: the skinny kernel's arrival counters
// always sit in its first kLinCntBytes (one per tile; a split layer has
// fewer than 128 tiles), and every partial buffer after them, so that calls
// of different shapes sharing one workspace never write over each other's
// counters (which each call leaves at zero).
constexpr size_t kLinCntBytes = 1024;

// Bytes of workspace a skinny split needs: the counters, then the partial tiles.
size_t skinny_ws_bytes(int N, int S) {
  const size_t tiles = (N + 15) / 16;
  return S > 1 ? kLinCntBytes + tiles * S * 256 * sizeof(float) : 0;
}

// a.kz: K range of one split (K when S == 1); a.part: partials; cnt: counters;
// a.cand (no LN): argmax candidates
int launch_skinny(const LinArgs& a, const float* c1, bool ln, int S, unsigned* cnt,
                  hipStream_t s) {
  const int st = skinny_steps(a.kz);
  const int nw = a.kz / (16 * st);
  const size_t lds = (size_t)nw * (256 + 32) * sizeof(float);
  const dim3 grid((a.N + 15) / 16, S);
  const bool cand = a.cand != nullptr;
#define SKV_SK(S_)                                                                          \
  if (st == S_) {                                                                           \
    if (ln)                                                                                 \
      hipLaunchKernelGGL((k_linear_skinny<S_, true>), grid, dim3(nw * 64), lds, s, a, c1,      \
                         cnt);                                                               \
    else if (cand)                                                                          \
      hipLaunchKernelGGL((k_linear_skinny<S_, false, true>), grid, dim3(nw * 64), lds, s, a, \
                         c1, cnt);                                                           \
    else                                                                                    \
      hipLaunchKernelGGL((k_linear_skinny<S_, false>), grid, dim3(nw * 64), lds, s, a, c1,     \
                         cnt);                                                               \
  }
  SKV_SK(3) SKV_SK(4) SKV_SK(6) SKV_SK(8) SKV_SK(12)
#undef SKV_SK
  return check_launch("skv_linear");
}

// skv_linear_pack: float4 p of the packed copy is lane l = p % 64 of 16-k
// step s = (p / 64) % (K / 16) of tile t = p / (64 K / 16): w[16 t + l % 16,
// 16 s + 4 (l / 16) .. + 3], zero past row N.
__global__ __launch_bounds__(256) void k_pack_mfma(float* __restrict__ wp,
                                                   const float* __restrict__ w, int N, int K,
                                                   size_t total4) {
  const size_t p = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= total4) return;
  const int l = (int)(p & 63);
  const size_t ts = p >> 6;
  const int steps = K / 16;
  const int s = (int)(ts % steps);
  const size_t t = ts / steps;
  const size_t n = t * 16 + (l & 15);
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (n < (size_t)N) v = *reinterpret_cast<const float4*>(w + n * K + 16 * s + 4 * (l >> 4));
  *reinterpret_cast<float4*>(wp + p * 4) = v;
}

// LayerNorm folding for k_linear_skinny: one workgroup per weight row n,
// sums in double in a fixed order.
__global__ __launch_bounds__(256) void k_fold_ln(float* __restrict__ wf, float* __restrict__ c1,
                                                 float* __restrict__ c2,
                                                 const float* __restrict__ w,
                                                 const float* __restrict__ g,
                                                 const float* __restrict__ b,
                                                 const float* __restrict__ bias, int K) {
  __shared__ double s1[256], s2[256];
  const int n = blockIdx.x, t = threadIdx.x;
  double a1 = 0.0, a2 = 0.0;
  for (int k = t; k < K; k += 256) {
    const float wv = w[(size_t)n * K + k];
    const float f = g[k] * wv;
    wf[(size_t)n * K + k] = f;
    a1 += (double)f;
    a2 += (double)b[k] * (double)wv;
  }
  s1[t] = a1;
  s2[t] = a2;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (t < o) {
      s1[t] += s1[t + o];
      s2[t] += s2[t + o];
    }
    __syncthreads();
  }
  if (t == 0) {
    c1[n] = (float)s1[0];
    c2[n] = (float)(s2[0] + (bias ? (double)bias[n] : 0.0));
  }
}

// Split-K finish: y = act(bias + sum of the S partials, in order) + res, one
// thread per output element.
__global__ __launch_bounds__(256) void k_linear_reduce(LinArgs a, int S) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)a.M * a.N) return;
  const int m = (int)(i / a.N), nn = (int)(i - (size_t)m * a.N);
  float v = a.bias ? a.bias[nn] : 0.f;
  for (int z = 0; z < S; ++z) v += a.part[((size_t)z * a.M + m) * a.N + nn];
  if (a.act == 1) v = gelu_tanh(v);
  size_t o = i;
  if (a.split > 0) {
    const int seg = nn / a.split;
    o = ((size_t)seg * a.M + m) * a.split + (nn - seg * a.split);
  }
  if (a.res) v += a.res[o];
  a.y[o] = v;
}

// Split count along K for a projection: narrow ones (fewer than ~160
// workgroups of 16 columns x 64 rows) leave most CUs idle, and a CU's weight
// stream is capped (~15-20 GB/s measured), so K is split until about 256
// workgroups run, keeping at least 16 steps (256 k) per split. Only long K
// (>= 2048) gains: measured on MI355X, the 16 x 768 x 3072 projection went
// from 13.5 to 10.3 us, while at K = 768 or 1024 the reduce launch costs more
// than the split saves.
int linear_splits(int M, int N, int K) {
  const long wgs = (long)((N + 15) / 16) * ((M + kLinRowsPerBlock - 1) / kLinRowsPerBlock);
  const int ksteps = (K + 15) / 16;
  if (wgs >= 160 || ksteps < 128) return 1;
  int S = (int)((256 + wgs - 1) / wgs);
  if (S > ksteps / 16) S = ksteps / 16;
  const int kz = (ksteps + S - 1) / S;  // steps per split; drop empty splits
  return (ksteps + kz - 1) / kz;
}

// ---------------------------------------------------------------------------
// argmax over each row (first index on ties), one workgroup per row
// ---------------------------------------------------------------------------
constexpr int kArgCols = 2048;  // columns per argmax workgroup (8 per thread)

__device__ __forceinline__ void block_better(float& bv, int& bi) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    better(bv, bi, ov, oi);
  }
}

// grid (slices, M): each workgroup finds the first maximum of its 2048-column
// slice of row m, all eight loads of a thread in flight at once. With one
// slice the winner is the answer; otherwise it goes to the candidate arrays
// and k_argmax_pick chooses among the slices in a second launch. (A last-
// arriving workgroup could pick instead, but its device-scope fence costs
// every one of the ~400 workgroups an L2 write-back, serialized per XCD:
// 18 us per call against 6 us for the two launches, measured on MI355X.)
__global__ __launch_bounds__(256) void k_argmax(int32_t* __restrict__ out,
                                                const float* __restrict__ x, int n,
                                                float* __restrict__ cand_v,
                                                int* __restrict__ cand_i) {
  __shared__ float sv[4];
  __shared__ int si[4];
  const int sl = blockIdx.x, m = blockIdx.y, ns = gridDim.x;
  const float* xr = x + (size_t)m * n;
  const int c0 = sl * kArgCols, c1 = min(n, c0 + kArgCols);
  float v[kArgCols / 256];
#pragma unroll
  for (int u = 0; u < kArgCols / 256; ++u) v[u] = xr[min(c0 + (int)threadIdx.x + 256 * u, c1 - 1)];
  float bv = -INFINITY;
  int bi = n;  // larger than any index: loses every tie
#pragma unroll
  for (int u = 0; u < kArgCols / 256; ++u) {
    const int j = c0 + threadIdx.x + 256 * u;
    if (j < c1) better(bv, bi, v[u], j);
  }
  block_better(bv, bi);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[w] = bv;
    si[w] = bi;
  }
  __syncthreads();
  if (threadIdx.x != 0) return;
  for (int i = 1; i < 4; ++i) better(bv, bi, sv[i], si[i]);
  if (ns == 1) {
    out[m] = bi < n ? bi : 0;  // a row of NaN only: token 0
  } else {
    cand_v[(size_t)m * ns + sl] = bv;
    cand_i[(size_t)m * ns + sl] = bi;
  }
}

// one wavefront per row: the first maximum over the slices' candidates
__global__ __launch_bounds__(64) void k_argmax_pick(int32_t* __restrict__ out,
                                                    const float* __restrict__ cand_v,
                                                    const int* __restrict__ cand_i, int ns, int n) {
  const int m = blockIdx.x;
  float bv = -INFINITY;
  int bi = n;
  for (int k = threadIdx.x; k < ns; k += 64)
    better(bv, bi, cand_v[(size_t)m * ns + k], cand_i[(size_t)m * ns + k]);
  block_better(bv, bi);
  if (threadIdx.x == 0) out[m] = bi < n ? bi : 0;
}

// ---------------------------------------------------------------------------
// next input token of every sequence: the next prompt token while the
// sequence is still inside its prompt, else the previous step's argmax. The
// chosen token is also recorded at its position in the sequence buffer.
// ---------------------------------------------------------------------------
// Retirement of a finished row (stop given): once the token at position
// stop[b] - 1 is recorded, every layer's fill of row b becomes -1, which the
// decode kernels treat as an empty row with no append and no advance, and
// the next-token kernels as a row that records nothing: the rest of the
// batch's steps read none of its cache.
__device__ __forceinline__ void retire_row(const int32_t* __restrict__ stop,
                                           int32_t* __restrict__ lens_all, int n_layers, int B,
                                           int b, int p) {
  if (stop != nullptr && p >= 0 && p >= stop[b] - 1)
    for (int li = 0; li < n_layers; ++li) lens_all[(size_t)li * B + b] = -1;
}

// Deferred fill advance (adv given): when the previous step's attention
// appended without advancing (adv[b] = 1), every layer's fill of row b moves
// past that token here, before anything of this step reads it; adv[b] is then
// set for this step's append. Returns the row's fill.
__device__ __forceinline__ int advance_row(int32_t* __restrict__ adv,
                                           int32_t* __restrict__ lens_all, int n_layers, int B,
                                           int b, int p, int cap) {
  if (adv[b] != 0 && p >= 0 && p < cap) {
    ++p;
    for (int li = 0; li < n_layers; ++li) lens_all[(size_t)li * B + b] = p;
  }
  adv[b] = 1;
  return p;
}

__global__ void k_next_tokens(int32_t* __restrict__ ids, int32_t* __restrict__ seq,
                              const int32_t* __restrict__ argmax_prev,
                              const int32_t* __restrict__ prompt,
                              const int32_t* __restrict__ prompt_len,
                              const int32_t* __restrict__ pos, int B, int max_prompt,
                              int seq_cap, const int32_t* __restrict__ stop,
                              int32_t* __restrict__ lens_all, int n_layers,
                              int32_t* __restrict__ adv) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  int p = pos[b];
  if (adv != nullptr) p = advance_row(adv, lens_all, n_layers, B, b, p, seq_cap);
  int t;
  if (p < prompt_len[b]) t = prompt[(size_t)b * max_prompt + min(max(p, 0), max_prompt - 1)];
  else t = argmax_prev[b];
  ids[b] = t;
  if (p >= 0 && p < seq_cap) seq[(size_t)b * seq_cap + p] = t;
  retire_row(stop, lens_all, n_layers, B, b, p);
}

// k_next_tokens and k_embed in one launch, with the argmax's last step: row
// b picks the first maximum over its n_cand (value, column) candidates (256
// threads), or reads argmax_prev[b] when n_cand is 0, applies the
// next-token rule above, records the token, and writes x[b] = embedding[t] +
// pos_table[pos] (no x when the embedding is null).
__global__ __launch_bounds__(256) void k_next_embed(
    float* __restrict__ x, int32_t* __restrict__ ids, int32_t* __restrict__ seq,
    const int32_t* __restrict__ argmax_prev, const float* __restrict__ cand, int n_cand,
    const int32_t* __restrict__ prompt, const int32_t* __restrict__ prompt_len,
    const int32_t* __restrict__ pos, int B, int max_prompt, int seq_cap,
    const float* __restrict__ emb, const float* __restrict__ pe, int d, int vocab, int ctx,
    const int32_t* __restrict__ stop, int32_t* __restrict__ lens_all, int n_layers,
    int32_t* __restrict__ adv) {
  __shared__ int s_t;
  __shared__ float s_bv[4];
  __shared__ int s_bi[4];
  const int b = blockIdx.x, tid = threadIdx.x;
  // The fill, the prompt length and the first 256 candidates are loaded
  // together, for every row (one inside its prompt ignores the candidates):
  // the candidates then arrive with the fill instead of one round trip after
  // it.
  // the fill after a deferred advance (every thread computes it; thread 0
  // writes it back after the block's last read of pos and adv)
  const int p0 = pos[b];
  const bool moves = adv != nullptr && adv[b] != 0 && p0 >= 0 && p0 < seq_cap;
  const int p = moves ? p0 + 1 : p0;
  const int plen = prompt_len[b];
  float bv = -INFINITY;
  int bi = vocab;
  const float* cv = cand + (size_t)b * n_cand;
  const int* ci = reinterpret_cast<const int*>(cand + (size_t)B * n_cand) + (size_t)b * n_cand;
  if (tid < n_cand) {
    bv = cv[tid];
    bi = ci[tid];
  }
  for (int k = tid + 256; k < n_cand; k += 256) better(bv, bi, cv[k], ci[k]);
  const bool in_prompt = p < plen;  // uniform
  if (n_cand > 0) {
    // the first maximum over the row's candidates, all 256 threads
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float ov = __shfl_xor(bv, o);
      const int oi = __shfl_xor(bi, o);
      better(bv, bi, ov, oi);
    }
    if ((tid & 63) == 0) {
      s_bv[tid >> 6] = bv;
      s_bi[tid >> 6] = bi;
    }
    __syncthreads();
  }
  if (adv != nullptr) __syncthreads();  // uniform: every thread has read pos[b] and adv[b]
  if (tid == 0) {
    if (adv != nullptr) {
      if (moves)
        for (int li = 0; li < n_layers; ++li) lens_all[(size_t)li * B + b] = p;
      adv[b] = 1;
    }
    int t;
    if (in_prompt) {
      t = prompt[(size_t)b * max_prompt + min(max(p, 0), max_prompt - 1)];
    } else if (n_cand > 0) {
      float bv = s_bv[0];
      int bi = s_bi[0];
      for (int w = 1; w < 4; ++w) better(bv, bi, s_bv[w], s_bi[w]);
      t = bi < vocab ? bi : 0;  // a row of NaN only: token 0
    } else {
      t = argmax_prev[b];
    }
    ids[b] = t;
    if (p >= 0 && p < seq_cap) seq[(size_t)b * seq_cap + p] = t;
    s_t = t;
    retire_row(stop, lens_all, n_layers, B, b, p);
  }
  if (emb == nullptr) return;  // uniform
  __syncthreads();
  const int id = min(max(s_t, 0), vocab - 1);
  const int pp = min(max(p, 0), ctx - 1);
  for (int j = tid; j < d; j += blockDim.x)
    x[(size_t)b * d + j] = emb[(size_t)id * d + j] + pe[(size_t)pp * d + j];
}

// y[m, :] = x[rows[m], :]; rows are clamped into [0, n_rows).
__global__ __launch_bounds__(256) void k_gather_rows(float* __restrict__ y,
                                                     const float* __restrict__ x,
                                                     const int32_t* __restrict__ rows, int d,
                                                     int n_rows) {
  const int m = blockIdx.x;
  const size_t r = (size_t)min(max(rows[m], 0), n_rows - 1);
  for (int j = threadIdx.x; j < d; j += blockDim.x) y[(size_t)m * d + j] = x[r * d + j];
}

}  // namespace
}  // namespace skv

using namespace skv;

extern "C" int skv_gather_rows(float* y, const float* x, const int32_t* rows, int M, int d,
                               int n_rows, skv_stream_t stream) {
  SKV_REQUIRE(y && x && rows, SKV_E_INVALID, "skv_gather_rows: null pointer argument");
  SKV_REQUIRE(M > 0 && d > 0 && n_rows > 0, SKV_E_INVALID, "skv_gather_rows: dims must be > 0");
  hipLaunchKernelGGL(k_gather_rows, dim3(M), dim3(256), 0, (hipStream_t)stream, y, x, rows, d,
                     n_rows);
  return check_launch("skv_gather_rows");
}

extern "C" int skv_embed(float* x, const int32_t* ids, const int32_t* pos, const float* embedding,
                         const float* pos_table, int M, int d, int vocab, int ctx,
                         skv_stream_t stream) {
  SKV_REQUIRE(x && ids && pos && embedding && pos_table, SKV_E_INVALID,
              "skv_embed: null pointer argument");
  SKV_REQUIRE(M > 0 && d > 0 && vocab > 0 && ctx > 0, SKV_E_INVALID, "skv_embed: dims must be > 0");
  hipLaunchKernelGGL(k_embed, dim3(M), dim3(256), 0, (hipStream_t)stream, x, ids, pos, embedding,
                     pos_table, d, vocab, ctx);
  return check_launch("skv_embed");
}

extern "C" int skv_layernorm(float* y, const float* x, const float* gamma, const float* beta,
                             int M, int d, float eps, skv_stream_t stream) {
  SKV_REQUIRE(y && x && gamma && beta, SKV_E_INVALID, "skv_layernorm: null pointer argument");
  SKV_REQUIRE(M > 0 && d > 0, SKV_E_INVALID, "skv_layernorm: dims must be > 0");
  SKV_REQUIRE(d <= 256 * kLnMaxPerThread, SKV_E_UNSUPPORTED, "skv_layernorm: d=%d > %d", d,
              256 * kLnMaxPerThread);
  hipLaunchKernelGGL(k_layernorm, dim3(M), dim3(256), 0, (hipStream_t)stream, y, x, gamma, beta,
                     d, eps);
  return check_launch("skv_layernorm");
}

extern "C" size_t skv_linear_workspace_bytes(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  // the GEMM path (more than one 64-row tile): LayerNorm row statistics
  if (M > kLinRowsPerBlock) return kLinCntBytes + (size_t)M * 2 * sizeof(float);
  // the skinny kernel's split and the LN path's k_linear split (either may
  // run for these sizes), after the counters
  const size_t sk = M <= 16 && skinny_steps(K) > 0 ? skinny_ws_bytes(N, skinny_splits(M, N, K)) : 0;
  const int S = linear_splits(M, N, K);
  const size_t kl = S > 1 ? kLinCntBytes + (size_t)S * M * N * sizeof(float) : 0;
  return sk > kl ? sk : kl;
}

extern "C" int skv_linear(float* y, const float* x, const float* w_t, const float* bias,
                          const float* residual, const float* ln_gamma, const float* ln_beta,
                          float ln_eps, int M, int N, int K, int activation, int split_cols,
                          void* ws, size_t ws_bytes, skv_stream_t stream) {
  SKV_REQUIRE(y && x && w_t, SKV_E_INVALID, "skv_linear: null pointer argument");
  SKV_REQUIRE(M > 0 && N > 0 && K > 0, SKV_E_INVALID, "skv_linear: dims must be > 0");
  SKV_REQUIRE(K % 4 == 0, SKV_E_UNSUPPORTED, "skv_linear: K=%d must be a multiple of 4", K);
  SKV_REQUIRE(activation == 0 || activation == 1, SKV_E_INVALID, "skv_linear: bad activation");
  SKV_REQUIRE(split_cols >= 0 && (split_cols == 0 || N % split_cols == 0), SKV_E_INVALID,
              "skv_linear: N=%d is not a multiple of split_cols=%d", N, split_cols);
  SKV_REQUIRE((ln_gamma == nullptr) == (ln_beta == nullptr), SKV_E_INVALID,
              "skv_linear: LayerNorm needs both gamma and beta");
  // Many rows (a prompt's prefill): the tiled GEMM, bound by the products
  // rather than by the weight stream.
  if (M > kLinRowsPerBlock) {
    const bool room = ws != nullptr && ws_bytes >= kLinCntBytes + (size_t)M * 2 * sizeof(float);
    float* stats = room ? reinterpret_cast<float*>(static_cast<char*>(ws) + kLinCntBytes) : nullptr;
    return gemm_linear(y, x, w_t, bias, residual, ln_gamma, ln_beta, ln_eps, M, N, K, activation,
                       split_cols, stats, (hipStream_t)stream);
  }
  // One row tile over many columns (the tied logits): k_linear_wide.
  {
    const int col_tiles = (N + 15) / 16;
    const int per_wg = (col_tiles + kNumCUs - 1) / kNumCUs;
    const int us = K / 64;
    if (M <= 16 && split_cols == 0 && col_tiles >= 1024 && K % 64 == 0 &&
        per_wg <= kWideMaxTiles && (us == 8 || us == 12 || us == 16)) {
      LinArgs a{y, x, w_t, bias, residual, ln_gamma, ln_beta, ln_eps, M, N, K, activation, 0, K,
                nullptr};
      const size_t lds = ((size_t)16 * (K + 4) + (size_t)per_wg * 4 * 64 * 4) * sizeof(float);
      const bool ln = ln_gamma != nullptr;
      hipStream_t s = (hipStream_t)stream;
#define SKV_WIDE(U, L)                                                                            if (us == U && ln == L)                                                                           hipLaunchKernelGGL((k_linear_wide<U, L>), dim3(kNumCUs), dim3(kWideWaves * 64), lds, s, a,                        col_tiles);
      SKV_WIDE(8, false) SKV_WIDE(8, true) SKV_WIDE(12, false) SKV_WIDE(12, true)
      SKV_WIDE(16, false) SKV_WIDE(16, true)
#undef SKV_WIDE
      return check_launch("skv_linear");
    }
  }
  // One row tile without LayerNorm, K a multiple of 48..192 (the decode
  // step's attention output and MLP down projections): k_linear_skinny.
  if (M <= 16 && ln_gamma == nullptr && skinny_steps(K) > 0) {
    int S = skinny_splits(M, N, K);
    if (S > 1 && (ws == nullptr || ws_bytes < skinny_ws_bytes(N, S))) S = 1;
    if (S > 1 || skinny_splits(M, N, K) == 1) {
      char* wsb = static_cast<char*>(ws);
      LinArgs a{y, x, w_t, bias, residual, nullptr, nullptr, 0.f, M, N, K, activation,
                split_cols, K / S, S > 1 ? reinterpret_cast<float*>(wsb + kLinCntBytes) : nullptr};
      return launch_skinny(a, nullptr, false, S, S > 1 ? reinterpret_cast<unsigned*>(wsb) : nullptr,
                           (hipStream_t)stream);
    }
  }
  const int ksteps = (K + 15) / 16;
  // split K when the caller gave room for the partials
  int S = linear_splits(M, N, K);
  if (S > 1 && (ws == nullptr || ws_bytes < kLinCntBytes + (size_t)S * M * N * sizeof(float)))
    S = 1;
  const int kz_steps = (ksteps + S - 1) / S;
  LinArgs a{y, x, w_t, bias, residual, ln_gamma, ln_beta, ln_eps, M, N, K, activation,
            split_cols, S > 1 ? kz_steps * 16 : K,
            S > 1 ? reinterpret_cast<float*>(static_cast<char*>(ws) + kLinCntBytes) : nullptr};
  const int col_tiles = (N + 15) / 16;
  const int tiles = M >= kLinRowsPerBlock ? 4 : (M + 15) / 16;
  // Wavefronts per workgroup and 16-k steps per wavefront and pass, measured
  // on MI355X:
  //  - one row tile (M <= 16) and 512 < K <= 768: 8 wavefronts of 6 steps,
  //    one pass (16 x 768 -> 768: 5.6 -> 4.8 us; the 16 x 768 -> 50304
  //    logits: 38.8 -> 36.4 us);
  //  - other narrow layers (few 16-column tiles, one CU each) split their K
  //    range over up to 16 wavefronts of at most 4 steps: deeper passes gain
  //    nothing, since a CU's weight stream is capped;
  //  - the wide logits with more row tiles use 8 wavefronts of 3 steps (3
  //    beat 4 and 12 by keeping more workgroups resident).
  // Steps never exceed what fits the registers without spilling (checked
  // with the compiler's resource report: per step, w and x take
  // (1 + TILES) * 4 registers and LN's gamma and beta 8 more).
  const bool wide = col_tiles >= 1024;
  const bool ln = ln_gamma != nullptr;
  int nw, max_steps;
  if (tiles == 1 && kz_steps > 32 && kz_steps <= 48) {
    nw = 8;  // 6 steps (5 would have no kernel; the extra steps are masked)
    max_steps = 6;
  } else {
    nw = wide ? 8 : (kz_steps < kLinMaxWaves ? kz_steps : kLinMaxWaves);
    max_steps = wide ? 3 : ln ? (tiles == 1 ? 4 : tiles == 2 ? 3 : 2) : (tiles == 4 ? 3 : 4);
  }
  nw = nw < tiles ? tiles : nw;  // the epilogue gives each wavefront at most 4 of the 4 TILES slots
  int steps = max_steps == 6 ? 6 : (kz_steps + nw - 1) / nw;
  steps = steps > max_steps ? max_steps : steps;
  dim3 grid(col_tiles, (M + kLinRowsPerBlock - 1) / kLinRowsPerBlock, S);
  const size_t lds = (size_t)nw * tiles * 64 * 4 * sizeof(float);
  hipStream_t s = (hipStream_t)stream;
  bool launched = false;
  const bool spread = M > 4;  // more than one row tile implies it
#define SKV_LIN(T, S_, L, SP)                                                             \
  if (!launched && tiles == T && steps == S_ && ln == L && spread == SP) {                \
    hipLaunchKernelGGL((k_linear<T, S_, L, SP>), grid, dim3(nw * 64), lds, s, a);         \
    launched = true;                                                                      \
  }
#define SKV_LIN2(T, S_) SKV_LIN(T, S_, false, true) SKV_LIN(T, S_, true, true)
#define SKV_LIN1(S_) SKV_LIN2(1, S_) SKV_LIN(1, S_, false, false) SKV_LIN(1, S_, true, false)
  SKV_LIN1(1) SKV_LIN1(2) SKV_LIN1(3) SKV_LIN1(4) SKV_LIN1(6)
  SKV_LIN2(2, 1) SKV_LIN2(2, 2) SKV_LIN2(2, 3) SKV_LIN(2, 4, false, true)
  SKV_LIN2(3, 1) SKV_LIN2(3, 2) SKV_LIN(3, 3, false, true) SKV_LIN(3, 4, false, true)
  SKV_LIN2(4, 1) SKV_LIN2(4, 2) SKV_LIN(4, 3, false, true)
#undef SKV_LIN1
#undef SKV_LIN2
#undef SKV_LIN
  if (!launched)
    return set_error(SKV_E_UNSUPPORTED, "skv_linear: no kernel for %d row tiles x %d steps",
                     tiles, steps);
  int rc = check_launch("skv_linear");
  if (rc || S == 1) return rc;
  const size_t n_out = (size_t)M * N;
  hipLaunchKernelGGL(k_linear_reduce, dim3((unsigned)((n_out + 255) / 256)), dim3(256), 0, s, a,
                     S);
  return check_launch("skv_linear");
}

extern "C" int skv_linear_fold_ln(float* w_fold, float* c1, float* c2, const float* w_t,
                                  const float* ln_gamma, const float* ln_beta, const float* bias,
                                  int N, int K, skv_stream_t stream) {
  SKV_REQUIRE(w_fold && c1 && c2 && w_t && ln_gamma && ln_beta, SKV_E_INVALID,
              "skv_linear_fold_ln: null pointer argument");
  SKV_REQUIRE(N > 0 && K > 0, SKV_E_INVALID, "skv_linear_fold_ln: dims must be > 0");
  SKV_REQUIRE(w_fold != w_t, SKV_E_INVALID, "skv_linear_fold_ln: w_fold may not alias w_t");
  hipLaunchKernelGGL(k_fold_ln, dim3(N), dim3(256), 0, (hipStream_t)stream, w_fold, c1, c2, w_t,
                     ln_gamma, ln_beta, bias, K);
  return check_launch("skv_linear_fold_ln");
}

extern "C" int skv_linear_folded(float* y, const float* x, const float* w_fold, const float* c1,
                                 const float* c2, const float* residual, float ln_eps, int M,
                                 int N, int K, int activation, int split_cols,
                                 skv_stream_t stream) {
  SKV_REQUIRE(y && x && w_fold && c1 && c2, SKV_E_INVALID,
              "skv_linear_folded: null pointer argument");
  SKV_REQUIRE(M > 0 && N > 0 && K > 0, SKV_E_INVALID, "skv_linear_folded: dims must be > 0");
  SKV_REQUIRE(activation == 0 || activation == 1, SKV_E_INVALID,
              "skv_linear_folded: bad activation");
  SKV_REQUIRE(split_cols >= 0 && (split_cols == 0 || N % split_cols == 0), SKV_E_INVALID,
              "skv_linear_folded: N=%d is not a multiple of split_cols=%d", N, split_cols);
  SKV_REQUIRE(M <= 16, SKV_E_UNSUPPORTED, "skv_linear_folded: M=%d > 16 rows", M);
  SKV_REQUIRE(skinny_steps(K) > 0, SKV_E_UNSUPPORTED,
              "skv_linear_folded: K=%d is not 16 * s * w for s in {3,4,6,8,12}, 4 <= w <= 16", K);
  LinArgs a{y, x, w_fold, c2, residual, nullptr, nullptr, ln_eps, M, N, K, activation,
            split_cols, K, nullptr};
  return launch_skinny(a, c1, true, 1, nullptr, (hipStream_t)stream);
}

extern "C" size_t skv_linear_packed_bytes(int N, int K) {
  if (N <= 0 || K <= 0 || K % 16) return 0;
  return (size_t)((N + 15) / 16) * 16 * K * sizeof(float);
}

extern "C" int skv_linear_pack(float* w_packed, const float* w_t, int N, int K,
                               skv_stream_t stream) {
  SKV_REQUIRE(w_packed && w_t, SKV_E_INVALID, "skv_linear_pack: null pointer argument");
  SKV_REQUIRE(N > 0 && K > 0 && K % 16 == 0, SKV_E_INVALID,
              "skv_linear_pack: N=%d, K=%d (K must be a positive multiple of 16)", N, K);
  const size_t total4 = skv_linear_packed_bytes(N, K) / 16;
  hipLaunchKernelGGL(k_pack_mfma, dim3((unsigned)((total4 + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, w_packed, w_t, N, K, total4);
  return check_launch("skv_linear_pack");
}

extern "C" int skv_linear_packed(float* y, const float* x, const float* w_packed,
                                 const float* bias, const float* residual, int M, int N, int K,
                                 int activation, float* argmax_cand, skv_stream_t stream) {
  SKV_REQUIRE(y && x && w_packed, SKV_E_INVALID, "skv_linear_packed: null pointer argument");
  SKV_REQUIRE(M > 0 && N > 0 && K > 0, SKV_E_INVALID, "skv_linear_packed: dims must be > 0");
  SKV_REQUIRE(activation == 0 || activation == 1, SKV_E_INVALID,
              "skv_linear_packed: bad activation");
  const int col_tiles = (N + 15) / 16;
  const int per_wg = (col_tiles + kNumCUs - 1) / kNumCUs;
  const int us = K / 64;
  SKV_REQUIRE(M <= 16 && K % 64 == 0 && (us == 8 || us == 12 || us == 16) &&
                  col_tiles >= 1024 && per_wg <= kWideMaxTiles,
              SKV_E_UNSUPPORTED,
              "skv_linear_packed: M=%d N=%d K=%d (needs M <= 16, K in {512, 768, 1024}, "
              "16384 <= N <= 65536)", M, N, K);
  LinArgs a{y, x, w_packed, bias, residual, nullptr, nullptr, 0.f, M, N, K, activation, 0, K,
            nullptr, argmax_cand};
  hipStream_t s = (hipStream_t)stream;
  // 16 wavefronts of K / 128 float4 a unit (eighths of a tile) where their
  // partials fit LDS beside x: a cold 154.5 MB stream measured 25.5 us at 16
  // wavefronts x 6 loads against 27.2 us at 8 x 12 on MI355X; else 8
  // wavefronts of quarters.
  const size_t x_lds = (size_t)16 * (K + 4) * sizeof(float);
  const size_t lds16 = x_lds + (size_t)per_wg * 8 * 64 * 4 * sizeof(float);
  const size_t lds8 = x_lds + (size_t)per_wg * 4 * 64 * 4 * sizeof(float);
  // the candidates' static LDS (16 wavefronts x 16 rows of value and column,
  // the arrival counter, padding to 16 bytes) comes on top of lds16
  const size_t cand_lds = argmax_cand ? 16 * 16 * 8 + 16 : 0;
  // The candidates are a kernel of their own (CAND): compiled into the plain
  // one, the unexecuted reduction left it ~5 us slower per call.
  const bool cand = argmax_cand != nullptr;
#define SKV_PKL(U, NWV, LDS)                                                                  \
  if (cand)                                                                                   \
    hipLaunchKernelGGL((k_linear_wide<U, false, true, NWV, true>), dim3(kNumCUs),             \
                       dim3(NWV * 64), LDS, s, a, col_tiles);                                 \
  else                                                                                        \
    hipLaunchKernelGGL((k_linear_wide<U, false, true, NWV, false>), dim3(kNumCUs),            \
                       dim3(NWV * 64), LDS, s, a, col_tiles);
  if (lds16 + cand_lds <= 160 * 1024) {
    if (K == 512) { SKV_PKL(4, 16, lds16) }
    else if (K == 768) { SKV_PKL(6, 16, lds16) }
    else { SKV_PKL(8, 16, lds16) }
  } else if (us == 8) {
    SKV_PKL(8, kWideWaves, lds8)
  } else if (us == 12) {
    SKV_PKL(12, kWideWaves, lds8)
  } else {
    SKV_PKL(16, kWideWaves, lds8)
  }
#undef SKV_PKL
  return check_launch("skv_linear_packed");
}

extern "C" size_t skv_argmax_workspace_bytes(int M, int N) {
  if (M <= 0 || N <= 0) return 0;
  const size_t ns = (N + kArgCols - 1) / kArgCols;
  return ns > 1 ? (size_t)M * 2 * ns * 4 : 0;
}

extern "C" int skv_argmax(int32_t* out, const float* x, int M, int N, void* ws, size_t ws_bytes,
                          skv_stream_t stream) {
  SKV_REQUIRE(out && x && M > 0 && N > 0, SKV_E_INVALID, "skv_argmax: bad arguments");
  SKV_REQUIRE(M <= 65535, SKV_E_UNSUPPORTED, "skv_argmax: M=%d too large", M);
  const size_t need = skv_argmax_workspace_bytes(M, N);
  SKV_REQUIRE(need == 0 || (ws && ws_bytes >= need), SKV_E_WORKSPACE,
              "skv_argmax: workspace %zu bytes < %zu required", ws_bytes, need);
  const int ns = (N + kArgCols - 1) / kArgCols;
  float* cv = static_cast<float*>(ws);  // M * ns candidate values, then their indices
  int* ci = reinterpret_cast<int*>(cv + (size_t)M * ns);
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(k_argmax, dim3(ns, M), dim3(256), 0, s, out, x, N, cv, ci);
  if (ns > 1) hipLaunchKernelGGL(k_argmax_pick, dim3(M), dim3(64), 0, s, out, cv, ci, ns, N);
  return check_launch("skv_argmax");
}

extern "C" size_t skv_linear_packed_cand_bytes(int M) {
  return M > 0 ? (size_t)M * kNumCUs * 8 : 0;
}

// The logits of a vocabulary too narrow for skv_linear_packed (C1: 256 from
// 256): skv_linear's one-tile-per-workgroup kernel (split K as skv_linear
// splits it when the workspace allows), with the candidates in its epilogue,
// so the step needs no argmax launch.
extern "C" int skv_linear_cand(float* y, const float* x, const float* w_t, const float* bias,
                               int M, int N, int K, float* argmax_cand, void* ws,
                               size_t ws_bytes, skv_stream_t stream) {
  SKV_REQUIRE(y && x && w_t && argmax_cand, SKV_E_INVALID, "skv_linear_cand: null pointer argument");
  SKV_REQUIRE(M > 0 && N > 0 && K > 0, SKV_E_INVALID, "skv_linear_cand: dims must be > 0");
  SKV_REQUIRE(M <= 16 && skinny_steps(K) > 0, SKV_E_UNSUPPORTED,
              "skv_linear_cand: M=%d K=%d (needs M <= 16 and K = 16 s w, s in {3, 4, 6, 8, 12}, "
              "4 <= w <= 16)", M, K);
  int S = skinny_splits(M, N, K);
  if (S > 1 && (ws == nullptr || ws_bytes < skinny_ws_bytes(N, S))) S = 1;
  char* wsb = static_cast<char*>(ws);
  LinArgs a{y, x, w_t, bias, nullptr, nullptr, nullptr, 0.f, M, N, K, 0, 0, K / S,
            S > 1 ? reinterpret_cast<float*>(wsb + kLinCntBytes) : nullptr, argmax_cand};
  return launch_skinny(a, nullptr, false, S, S > 1 ? reinterpret_cast<unsigned*>(wsb) : nullptr,
                       (hipStream_t)stream);
}

extern "C" size_t skv_linear_cand_bytes(int M, int N, int K) {
  if (M <= 0 || M > 16 || N <= 0 || K <= 0 || skinny_steps(K) == 0) return 0;
  return (size_t)M * ((N + 15) / 16) * 8;
}

extern "C" int skv_next_embed(float* x, int32_t* ids, int32_t* seq, const int32_t* argmax_prev,
                              const float* cand, int n_cand, const int32_t* prompt,
                              const int32_t* prompt_len, const int32_t* pos, int B,
                              int max_prompt, int seq_cap, const float* embedding,
                              const float* pos_table, int d, int vocab, int ctx,
                              const int32_t* stop, int32_t* lens_all, int n_layers,
                              int32_t* adv, skv_stream_t stream) {
  SKV_REQUIRE(ids && seq && prompt && prompt_len && pos, SKV_E_INVALID,
              "skv_next_embed: null pointer argument");
  SKV_REQUIRE((stop == nullptr && adv == nullptr) || (lens_all != nullptr && n_layers > 0),
              SKV_E_INVALID,
              "skv_next_embed: retiring rows or advancing fills needs lens_all and n_layers > 0");
  SKV_REQUIRE(B > 0 && max_prompt > 0 && seq_cap > 0 && vocab > 0 && n_cand >= 0, SKV_E_INVALID,
              "skv_next_embed: bad sizes");
  SKV_REQUIRE(n_cand > 0 ? cand != nullptr : argmax_prev != nullptr, SKV_E_INVALID,
              "skv_next_embed: candidates or the previous argmax needed");
  SKV_REQUIRE(embedding == nullptr || (x && pos_table && d > 0 && ctx > 0), SKV_E_INVALID,
              "skv_next_embed: embedding needs x, pos_table, d and ctx");
  hipLaunchKernelGGL(k_next_embed, dim3(B), dim3(256), 0, (hipStream_t)stream, x, ids, seq,
                     argmax_prev, cand, n_cand, prompt, prompt_len, pos, B, max_prompt, seq_cap,
                     embedding, pos_table, d, vocab, ctx, stop, lens_all, n_layers, adv);
  return check_launch("skv_next_embed");
}

extern "C" int skv_next_tokens(int32_t* ids, int32_t* seq, const int32_t* argmax_prev,
                               const int32_t* prompt, const int32_t* prompt_len,
                               const int32_t* pos, int B, int max_prompt, int seq_cap,
                               const int32_t* stop, int32_t* lens_all, int n_layers,
                               int32_t* adv, skv_stream_t stream) {
  SKV_REQUIRE(ids && seq && argmax_prev && prompt && prompt_len && pos, SKV_E_INVALID,
              "skv_next_tokens: null pointer argument");
  SKV_REQUIRE(B > 0 && max_prompt > 0 && seq_cap > 0, SKV_E_INVALID,
              "skv_next_tokens: dims must be > 0");
  SKV_REQUIRE((stop == nullptr && adv == nullptr) || (lens_all != nullptr && n_layers > 0),
              SKV_E_INVALID,
              "skv_next_tokens: retiring rows or advancing fills needs lens_all and n_layers > 0");
  hipLaunchKernelGGL(k_next_tokens, dim3((B + 255) / 256), dim3(256), 0, (hipStream_t)stream, ids,
                     seq, argmax_prev, prompt, prompt_len, pos, B, max_prompt, seq_cap, stop,
                     lens_all, n_layers, adv);
  return check_launch("skv_next_tokens");
}
