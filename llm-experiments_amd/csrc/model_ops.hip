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
// workgroup owns 16 output columns and up to 64 rows; its 4 wavefronts split
// K, each feeding one 16x16 tile per 16-row block, and the partial tiles are
// summed through LDS before the fused epilogue (bias, GELU, residual).
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
  int M, N, K;
  int act;      // 0 none, 1 gelu (tanh form)
  int split;    // > 0: column n goes to segment n / split of a [N/split][M][split] output
};

// Lane layout of v_mfma_f32_16x16x4_f32: operand A lane l holds
// (m = l % 16, k = l / 16), operand B holds (k = l / 16, n = l % 16), and
// result slot i holds (m = 4 * (l / 16) + i, n = l % 16). Within each step
// of 16 k the four MFMAs take k = k0 + 4 * (l / 16) + i for i = 0..3 from
// the same 16-byte load of x and of Wt (a consistent permutation of k).
__global__ __launch_bounds__(256) void k_linear(LinArgs a) {
  __shared__ float red[4][4][64][4];  // [wave][row tile][lane][slot]
  const int n0 = blockIdx.x * 16;
  const int m0 = blockIdx.y * kLinRowsPerBlock;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int lr = l & 15, lk = l >> 4;
  // K range of this wavefront, in steps of 16
  const int steps = (a.K + 15) / 16;
  const int per = (steps + 3) / 4;
  const int k_begin = wave * per * 16;
  const int k_end = min(a.K, (wave + 1) * per * 16);

  f32x4 acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int n = n0 + lr;
  const bool n_ok = n < a.N;
  const float* wrow = a.wt + (size_t)(n_ok ? n : 0) * a.K;
  int rows_here = min(kLinRowsPerBlock, a.M - m0);
  const int tiles = (rows_here + 15) / 16;

  for (int k = k_begin; k < k_end; k += 16) {
    const int kk = k + 4 * lk;
    const bool k_ok = kk < a.K;  // K % 4 == 0, so a 16-byte group is all in or all out
    const float4 w = (n_ok && k_ok) ? *reinterpret_cast<const float4*>(wrow + kk)
                                    : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (t < tiles) {
        const int m = m0 + t * 16 + lr;
        const float4 xv = (m < a.M && k_ok)
                              ? *reinterpret_cast<const float4*>(a.x + (size_t)m * a.K + kk)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.x, w.x, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.y, w.y, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.z, w.z, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.w, w.w, acc[t], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][t][l][i] = acc[t][i];
  __syncthreads();
  // thread -> (row tile t, lane ll): sums the 4 wavefronts' partial tiles
  const int t = threadIdx.x >> 6, ll = threadIdx.x & 63;
  if (t >= tiles) return;
  const int nn = n0 + (ll & 15);
  if (nn >= a.N) return;
  const float b = a.bias ? a.bias[nn] : 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + t * 16 + 4 * (ll >> 4) + i;
    if (m >= a.M) continue;
    float v = red[0][t][ll][i] + red[1][t][ll][i] + red[2][t][ll][i] + red[3][t][ll][i] + b;
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

__global__ __launch_bounds__(256) void k_argmax(int32_t* __restrict__ out,
                                                const float* __restrict__ x, int n) {
  __shared__ float sv[4];
  __shared__ int si[4];
  const int m = blockIdx.x;
  const float* xr = x + (size_t)m * n;
  float bv = -INFINITY;
  int bi = n;  // larger than any index: loses every tie
  for (int j = threadIdx.x; j < n; j += 256) better(bv, bi, xr[j], j);
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
    out[m] = bi < n ? bi : 0;  // a row of NaN/-inf only: token 0
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
                          const float* residual, int M, int N, int K, int activation,
                          int split_cols, skv_stream_t stream) {
  SKV_REQUIRE(y && x && w_t, SKV_E_INVALID, "skv_linear: null pointer argument");
  SKV_REQUIRE(M > 0 && N > 0 && K > 0, SKV_E_INVALID, "skv_linear: dims must be > 0");
  SKV_REQUIRE(K % 4 == 0, SKV_E_UNSUPPORTED, "skv_linear: K=%d must be a multiple of 4", K);
  SKV_REQUIRE(activation == 0 || activation == 1, SKV_E_INVALID, "skv_linear: bad activation");
  SKV_REQUIRE(split_cols >= 0 && (split_cols == 0 || N % split_cols == 0), SKV_E_INVALID,
              "skv_linear: N=%d is not a multiple of split_cols=%d", N, split_cols);
  SKV_REQUIRE((M + kLinRowsPerBlock - 1) / kLinRowsPerBlock <= 65535, SKV_E_UNSUPPORTED,
              "skv_linear: M=%d too large", M);
  LinArgs a{y, x, w_t, bias, residual, M, N, K, activation, split_cols};
  dim3 grid((N + 15) / 16, (M + kLinRowsPerBlock - 1) / kLinRowsPerBlock);
  hipLaunchKernelGGL(k_linear, grid, dim3(256), 0, (hipStream_t)stream, a);
  return check_launch("skv_linear");
}

extern "C" int skv_argmax(int32_t* out, const float* x, int M, int N, skv_stream_t stream) {
  SKV_REQUIRE(out && x && M > 0 && N > 0, SKV_E_INVALID, "skv_argmax: bad arguments");
  hipLaunchKernelGGL(k_argmax, dim3(M), dim3(256), 0, (hipStream_t)stream, out, x, N);
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
