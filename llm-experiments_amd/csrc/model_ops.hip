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
constexpr int kLinRowsPerBlock = 64;  // 4 tiles of 16 rows
constexpr int kLinMaxWaves = 16;      // wavefronts per workgroup, splitting K

__device__ __forceinline__ float gelu_tanh(float v) {
  const float k0 = 0.7978845608028654f;  // sqrt(2 / pi)
  return 0.5f * v * (1.f + tanhf(k0 * (v + 0.044715f * v * v * v)));
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
  extern __shared__ float red[];  // partial tiles of the W wavefronts (layout below)
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
__device__ __forceinline__ void better(float& bv, int& bi, float v, int i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

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
__global__ void k_next_tokens(int32_t* __restrict__ ids, int32_t* __restrict__ seq,
                              const int32_t* __restrict__ argmax_prev,
                              const int32_t* __restrict__ prompt,
                              const int32_t* __restrict__ prompt_len,
                              const int32_t* __restrict__ pos, int B, int max_prompt,
                              int seq_cap) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const int p = pos[b];
  int t;
  if (p < prompt_len[b]) t = prompt[(size_t)b * max_prompt + min(p, max_prompt - 1)];
  else t = argmax_prev[b];
  ids[b] = t;
  if (p >= 0 && p < seq_cap) seq[(size_t)b * seq_cap + p] = t;
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
  if (M > kLinRowsPerBlock) return (size_t)M * 2 * sizeof(float);
  const int S = linear_splits(M, N, K);
  return S > 1 ? (size_t)S * M * N * sizeof(float) : 0;
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
    const bool room = ws != nullptr && ws_bytes >= (size_t)M * 2 * sizeof(float);
    return gemm_linear(y, x, w_t, bias, residual, ln_gamma, ln_beta, ln_eps, M, N, K, activation,
                       split_cols, room ? static_cast<float*>(ws) : nullptr, (hipStream_t)stream);
  }
  const int ksteps = (K + 15) / 16;
  // split K when the caller gave room for the partials
  int S = linear_splits(M, N, K);
  if (S > 1 && (ws == nullptr || ws_bytes < (size_t)S * M * N * sizeof(float))) S = 1;
  const int kz_steps = (ksteps + S - 1) / S;
  LinArgs a{y, x, w_t, bias, residual, ln_gamma, ln_beta, ln_eps, M, N, K, activation,
            split_cols, S > 1 ? kz_steps * 16 : K, S > 1 ? static_cast<float*>(ws) : nullptr};
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

extern "C" int skv_next_tokens(int32_t* ids, int32_t* seq, const int32_t* argmax_prev,
                               const int32_t* prompt, const int32_t* prompt_len,
                               const int32_t* pos, int B, int max_prompt, int seq_cap,
                               skv_stream_t stream) {
  SKV_REQUIRE(ids && seq && argmax_prev && prompt && prompt_len && pos, SKV_E_INVALID,
              "skv_next_tokens: null pointer argument");
  SKV_REQUIRE(B > 0 && max_prompt > 0 && seq_cap > 0, SKV_E_INVALID,
              "skv_next_tokens: dims must be > 0");
  hipLaunchKernelGGL(k_next_tokens, dim3((B + 255) / 256), dim3(256), 0, (hipStream_t)stream, ids,
                     seq, argmax_prev, prompt, prompt_len, pos, B, max_prompt, seq_cap);
  return check_launch("skv_next_tokens");
}
