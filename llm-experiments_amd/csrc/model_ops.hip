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

// Split reductions: every workgroup of a group writes its partial result,
// then arrives on the group's counter; exactly one workgroup (the last to
// arrive) sees true, after all partials are visible to it, and resets the
// counter to zero for the next call. Counters must be zero before the first
// call. The last workgroup sums the partials in a fixed order, so results do
// not depend on arrival order.
__device__ __forceinline__ bool last_arrival(int* counter, int n) {
  __shared__ int is_last;
  __syncthreads();  // this workgroup's partial stores are issued
  if (threadIdx.x == 0) {
    __threadfence();  // release them device-wide (across XCDs)
    const int prev = atomicAdd(counter, 1);
    is_last = prev == n - 1;
    if (is_last) atomicExch(counter, 0);
  }
  __syncthreads();
  if (is_last) __threadfence();  // acquire the other workgroups' partials
  return is_last != 0;
}

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
};

// Lane layout of v_mfma_f32_16x16x4_f32: operand A lane l holds
// (m = l % 16, k = l / 16), operand B holds (k = l / 16, n = l % 16), and
// result slot i holds (m = 4 * (l / 16) + i, n = l % 16). Within each step
// of 16 k the four MFMAs take k = k0 + 4 * (l / 16) + i for i = 0..3 from
// the same 16-byte load of x and of Wt (a consistent permutation of k).
//
// The W wavefronts of a workgroup (W = blockDim / 64) split K in contiguous
// ranges, each keeping U weight loads in flight, and sum their tiles through
// LDS; no workgroup waits on another. Measured on MI355X (M = 16): a CU
// streams ~15-20 GB/s of weights whatever W and U are, so narrow layers
// (few 16-column tiles, one CU each) want many short-range wavefronts
// (W = 16, U = 2) and wide layers (the 50304-column logits) few long ones
// (W = 2, U = 8); a masked deep unroll costs extra time on small K. With ln_g set, each x row is layer-normalized as it is read
// (mean and 1/std of the workgroup's rows are computed first), which takes
// the LayerNorm launch out of the step.
template <int TILES, int U>
__global__ __launch_bounds__(kLinMaxWaves * 64) void k_linear(LinArgs a) {
  constexpr int kLinUnroll = U;
  extern __shared__ float red[];  // [W][TILES][64][4] partial tiles
  __shared__ float stat[kLinRowsPerBlock][2];
  const int NW = blockDim.x >> 6;
  const int n0 = blockIdx.x * 16;
  const int m0 = blockIdx.y * kLinRowsPerBlock;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int lr = l & 15, lk = l >> 4;
  const int rows = min(TILES * 16, a.M - m0);
  const bool ln = a.ln_g != nullptr;

  if (ln) {
    // Row statistics, one wavefront per row, in a single pass over values
    // shifted by the row's first element c (var = E[(x-c)^2] - E[x-c]^2 stays
    // well conditioned when |mean| >> std), so all loads are in flight at once.
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

  // K range of this wavefront, in steps of 16
  const int steps = (a.K + 15) / 16;
  const int per = (steps + NW - 1) / NW;
  const int k_begin = wave * per * 16;
  const int k_end = min(a.K, (wave + 1) * per * 16);

  f32x4 acc[TILES];
#pragma unroll
  for (int t = 0; t < TILES; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int n = n0 + lr;
  const bool n_ok = n < a.N;
  const float* wrow = a.wt + (size_t)(n_ok ? n : 0) * a.K;

  auto load_w = [&](int kk) {
    return (n_ok && kk < a.K) ? *reinterpret_cast<const float4*>(wrow + kk)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
  };
  auto fma_step = [&](int kk, const float4& w) {
    float4 g = make_float4(1.f, 1.f, 1.f, 1.f), bb = make_float4(0.f, 0.f, 0.f, 0.f);
    if (ln && kk < a.K) {
      g = *reinterpret_cast<const float4*>(a.ln_g + kk);
      bb = *reinterpret_cast<const float4*>(a.ln_b + kk);
    }
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      const int r = t * 16 + lr;
      float4 xv = (r < rows && kk < a.K)
                      ? *reinterpret_cast<const float4*>(a.x + (size_t)(m0 + r) * a.K + kk)
                      : make_float4(0.f, 0.f, 0.f, 0.f);
      if (ln && r < rows && kk < a.K) {
        const float mu = stat[r][0], rs = stat[r][1];
        xv.x = (xv.x - mu) * rs * g.x + bb.x;
        xv.y = (xv.y - mu) * rs * g.y + bb.y;
        xv.z = (xv.z - mu) * rs * g.z + bb.z;
        xv.w = (xv.w - mu) * rs * g.w + bb.w;
      }
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.x, w.x, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.y, w.y, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.z, w.z, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.w, w.w, acc[t], 0, 0, 0);
    }
  };
  // All (up to kLinUnroll) steps of a round issue their loads before any
  // MFMA; steps past this wavefront's range are masked to zero, so a short
  // range costs one round trip. K % 4 == 0: a 16-byte group at kk is either
  // wholly inside the range or past it.
  for (int k = k_begin; k < k_end; k += 16 * kLinUnroll) {
    float4 w[kLinUnroll];
#pragma unroll
    for (int u = 0; u < kLinUnroll; ++u) {
      const int kk = k + u * 16 + 4 * lk;
      w[u] = kk < k_end ? load_w(kk) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < kLinUnroll; ++u) {
      const int kk = k + u * 16 + 4 * lk;
      fma_step(kk < k_end ? kk : a.K, w[u]);  // kk = K marks a masked step
    }
  }
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[((wave * TILES + t) * 64 + l) * 4 + i] = acc[t][i];
  __syncthreads();
  // thread -> (row tile t, lane ll): sums the wavefronts' partial tiles
  if (threadIdx.x >= TILES * 64) return;
  const int t = threadIdx.x >> 6, ll = threadIdx.x & 63;
  if (t * 16 >= rows) return;
  const int nn = n0 + (ll & 15);
  if (nn >= a.N) return;
  const float b = a.bias ? a.bias[nn] : 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + t * 16 + 4 * (ll >> 4) + i;
    if (m >= a.M) continue;
    float v = b;
    for (int wv = 0; wv < NW; ++wv) v += red[((wv * TILES + t) * 64 + ll) * 4 + i];
    if (a.act == 1) v = gelu_tanh(v);
    size_t o;
    if (a.split > 0) {
      const int seg = nn / a.split;
      o = ((size_t)seg * a.M + m) * a.split + (nn - seg * a.split);
    } else {
      o = (size_t)m * a.N + nn;
    }
    if (a.res) v += a.res[o];
    a.y[o] = v;
  }
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

constexpr int kArgCols = 2048;  // columns per argmax workgroup

// grid (slices, M): each workgroup finds the first maximum of its slice of
// row m; the last slice to arrive picks the winner over the slices in order.
__global__ __launch_bounds__(256) void k_argmax(int32_t* __restrict__ out,
                                                const float* __restrict__ x, int n,
                                                float* __restrict__ cand_v,
                                                int* __restrict__ cand_i,
                                                int* __restrict__ counters) {
  __shared__ float sv[4];
  __shared__ int si[4];
  const int sl = blockIdx.x, m = blockIdx.y, ns = gridDim.x;
  const float* xr = x + (size_t)m * n;
  const int c0 = sl * kArgCols, c1 = min(n, c0 + kArgCols);
  float bv = -INFINITY;
  int bi = n;  // larger than any index: loses every tie
  for (int j = c0 + threadIdx.x; j < c1; j += 256) better(bv, bi, xr[j], j);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    better(bv, bi, ov, oi);
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[w] = bv;
    si[w] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < 4; ++i) better(bv, bi, sv[i], si[i]);
    cand_v[(size_t)m * ns + sl] = bv;
    cand_i[(size_t)m * ns + sl] = bi;
  }
  if (!last_arrival(counters + m, ns)) return;
  if (threadIdx.x == 0) {
    float v = -INFINITY;
    int i = n;
    for (int k = 0; k < ns; ++k) better(v, i, cand_v[(size_t)m * ns + k], cand_i[(size_t)m * ns + k]);
    out[m] = i < n ? i : 0;  // a row of NaN/-inf only: token 0
  }
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

}  // namespace
}  // namespace skv

using namespace skv;

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

extern "C" int skv_linear(float* y, const float* x, const float* w_t, const float* bias,
                          const float* residual, const float* ln_gamma, const float* ln_beta,
                          float ln_eps, int M, int N, int K, int activation, int split_cols,
                          skv_stream_t stream) {
  SKV_REQUIRE(y && x && w_t, SKV_E_INVALID, "skv_linear: null pointer argument");
  SKV_REQUIRE(M > 0 && N > 0 && K > 0, SKV_E_INVALID, "skv_linear: dims must be > 0");
  SKV_REQUIRE(K % 4 == 0, SKV_E_UNSUPPORTED, "skv_linear: K=%d must be a multiple of 4", K);
  SKV_REQUIRE(activation == 0 || activation == 1, SKV_E_INVALID, "skv_linear: bad activation");
  SKV_REQUIRE(split_cols >= 0 && (split_cols == 0 || N % split_cols == 0), SKV_E_INVALID,
              "skv_linear: N=%d is not a multiple of split_cols=%d", N, split_cols);
  SKV_REQUIRE((ln_gamma == nullptr) == (ln_beta == nullptr), SKV_E_INVALID,
              "skv_linear: LayerNorm needs both gamma and beta");
  SKV_REQUIRE((M + kLinRowsPerBlock - 1) / kLinRowsPerBlock <= 65535, SKV_E_UNSUPPORTED,
              "skv_linear: M=%d too large", M);
  LinArgs a{y, x, w_t, bias, residual, ln_gamma, ln_beta, ln_eps, M, N, K, activation,
            split_cols};
  const int col_tiles = (N + 15) / 16;
  // enough wavefronts per tile that narrow layers still fill the machine
  const bool wide = col_tiles >= 1024;
  const int nw = wide ? 2 : 16;
  const int tiles = M >= kLinRowsPerBlock ? 4 : (M + 15) / 16;
  dim3 grid(col_tiles, (M + kLinRowsPerBlock - 1) / kLinRowsPerBlock);
  const size_t lds = (size_t)nw * tiles * 64 * 4 * sizeof(float);
  hipStream_t s = (hipStream_t)stream;
#define SKV_LIN(T)                                                                           \
  if (wide) hipLaunchKernelGGL((k_linear<T, 8>), grid, dim3(nw * 64), lds, s, a);           \
  else hipLaunchKernelGGL((k_linear<T, 2>), grid, dim3(nw * 64), lds, s, a);
  switch (tiles) {
    case 1: SKV_LIN(1) break;
    case 2: SKV_LIN(2) break;
    case 3: SKV_LIN(3) break;
    default: SKV_LIN(4) break;
  }
#undef SKV_LIN
  return check_launch("skv_linear");
}

extern "C" size_t skv_argmax_workspace_bytes(int M, int N) {
  if (M <= 0 || N <= 0) return 0;
  const size_t ns = (N + kArgCols - 1) / kArgCols;
  return (size_t)M * (2 * ns + 1) * 4;
}

extern "C" int skv_argmax(int32_t* out, const float* x, int M, int N, void* ws, size_t ws_bytes,
                          skv_stream_t stream) {
  SKV_REQUIRE(out && x && M > 0 && N > 0, SKV_E_INVALID, "skv_argmax: bad arguments");
  SKV_REQUIRE(M <= 65535, SKV_E_UNSUPPORTED, "skv_argmax: M=%d too large", M);
  const size_t need = skv_argmax_workspace_bytes(M, N);
  SKV_REQUIRE(ws && ws_bytes >= need, SKV_E_WORKSPACE,
              "skv_argmax: workspace %zu bytes < %zu required", ws_bytes, need);
  const int ns = (N + kArgCols - 1) / kArgCols;
  int* cnt = static_cast<int*>(ws);  // M counters first, then the candidates
  float* cv = reinterpret_cast<float*>(cnt + M);
  int* ci = reinterpret_cast<int*>(cv + (size_t)M * ns);
  hipLaunchKernelGGL(k_argmax, dim3(ns, M), dim3(256), 0, (hipStream_t)stream, out, x, N, cv, ci,
                     cnt);
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
