// Projections over many rows (the model's prompt prefill): a tiled fp32
// GEMM on MFMA, y = act(LN(x) . w_t^T + bias) + residual, with the
// semantics of skv_linear (the reference's jnp.dot projections,
// simple-llm/src/jax_backend.py:110-129, 147, over every position of a
// window). skv_linear runs this kernel when a call has more than 64 rows;
// the decode step's few rows stay on k_linear (model_ops.hip), which is
// bound by reading the weights rather than by the products.
//
// Design: workgroup tile 128 rows x 128 output columns, 4 wavefronts of
// 64 x 64 (2 x 2 tiles of v_mfma_f32_32x32x2_f32), K in steps of 32. The x
// and w_t tiles of a step are K-contiguous rows in both operands; they go
// global -> registers -> LDS ([128][32 + 4] floats each: 16-byte reads of
// 16 consecutive rows hit distinct banks), and the next step's global
// loads are issued before the current step's products. A lane reads four
// consecutive k of its row with one 16-byte LDS load and feeds them to four
// MFMAs (k = 4*hf + t of each 8-k group, the same permutation for both
// operands). LayerNorm, when asked for, is applied to the x tile as it is
// staged, from per-row statistics computed by k_rowstats first (or, without
// a workspace to hold them, by each workgroup for its own 128 rows).
#include "skv_common.h"

namespace skv {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 128, kBN = 128, kBK = 32;
constexpr int kSP = kBK + 4;  // LDS row stride (floats)
constexpr int kThreads = 256;
constexpr int kLoads = kBM * kBK / 4 / kThreads;  // float4 per thread per operand (4)

__device__ __forceinline__ float gelu_tanh_g(float v) {
  const float k0 = 0.7978845608028654f;  // sqrt(2 / pi)
  return 0.5f * v * (1.f + tanhf(k0 * (v + 0.044715f * v * v * v)));
}

struct GemmArgs {
  float* y;
  const float* x;
  const float* wt;
  const float* bias;
  const float* res;
  const float* ln_g;   // LayerNorm of the x rows (NULL: none)
  const float* ln_b;
  const float* stats;  // [M][2] mean, 1/std of the x rows (with LN; NULL: computed here)
  float ln_eps;
  int M, N, K;
  int act;    // 0 none, 1 GELU (tanh form)
  int split;  // > 0: column n goes to segment n / split of a [N/split][M][split] output
};

// Row mean and 1/sqrt(var + eps) (population variance, jax_backend.py:78-82),
// one wavefront per row; sums of the values shifted by the row's first
// element.
__global__ __launch_bounds__(256) void k_rowstats(float* __restrict__ stats,
                                                  const float* __restrict__ x, int M, int K,
                                                  float eps) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
  if (row >= M) return;
  const float* xr = x + (size_t)row * K;
  const float c = xr[0];
  float s = 0.f, q = 0.f;
  for (int j = l; j < K; j += 64) {
    const float v = xr[j] - c;
    s += v;
    q += v * v;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    s += __shfl_xor(s, o);
    q += __shfl_xor(q, o);
  }
  if (l == 0) {
    const float ms = s / K;
    stats[(size_t)row * 2] = c + ms;
    stats[(size_t)row * 2 + 1] = 1.f / sqrtf(fmaxf(q / K - ms * ms, 0.f) + eps);
  }
}

template <bool LN>
__global__ __launch_bounds__(kThreads) void k_gemm(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) float sA[kBM * kSP];
  __shared__ __attribute__((aligned(16))) float sB[kBN * kSP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 31, hf = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;  // the wavefront's 64 x 64 quadrant
  const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;

  // staging: float4 e = tid + 256 u of a 128 x 32 tile is row e / 8, k 4 (e % 8)
  f32x4 ra[kLoads], rb[kLoads];
  float mu[LN ? kLoads : 1], rs[LN ? kLoads : 1];
  if constexpr (LN) {
    __shared__ float sstat[LN ? kBM : 1][2];
    const float* st = a.stats;
    if (st == nullptr) {
      // row statistics of this tile's rows, one wavefront per row (shifted by
      // the row's first element, as k_rowstats)
      for (int rr = wave; rr < kBM; rr += kThreads / 64) {
        const float* xr = a.x + (size_t)min(m0 + rr, a.M - 1) * a.K;
        const float c0 = xr[0];
        float sm = 0.f, sq = 0.f;
        for (int j = lane; j < a.K; j += 64) {
          const float v = xr[j] - c0;
          sm += v;
          sq += v * v;
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
          sm += __shfl_xor(sm, o);
          sq += __shfl_xor(sq, o);
        }
        if (lane == 0) {
          const float ms = sm / a.K;
          sstat[rr][0] = c0 + ms;
          sstat[rr][1] = 1.f / sqrtf(fmaxf(sq / a.K - ms * ms, 0.f) + a.ln_eps);
        }
      }
      __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      const int r = (tid + kThreads * u) >> 3;
      const int m = min(m0 + r, a.M - 1);
      mu[u] = st ? st[(size_t)m * 2] : sstat[r][0];
      rs[u] = st ? st[(size_t)m * 2 + 1] : sstat[r][1];
    }
  }
  // Global loads read clamped, in-bounds addresses; values past K are
  // zeroed afterwards (K % 4 == 0, so a float4 lies wholly inside or past K).
  auto load_tile = [&](int k0) {
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      const int e = tid + kThreads * u, r = e >> 3, kk = k0 + 4 * (e & 7);
      const int kc = min(kk, a.K - 4);
      ra[u] = *reinterpret_cast<const f32x4*>(a.x + (size_t)min(m0 + r, a.M - 1) * a.K + kc);
      rb[u] = *reinterpret_cast<const f32x4*>(a.wt + (size_t)min(n0 + r, a.N - 1) * a.K + kc);
    }
  };
  auto store_tile = [&](int k0) {
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      const int e = tid + kThreads * u, r = e >> 3, kq = 4 * (e & 7);
      const bool kin = k0 + kq < a.K;
      f32x4 va = ra[u], vb = rb[u];
      if constexpr (LN) {
        const int kc = min(k0 + kq, a.K - 4);
        const f32x4 g = *reinterpret_cast<const f32x4*>(a.ln_g + kc);
        const f32x4 bb = *reinterpret_cast<const f32x4*>(a.ln_b + kc);
#pragma unroll
        for (int t = 0; t < 4; ++t) va[t] = (va[t] - mu[u]) * rs[u] * g[t] + bb[t];
      }
      if (!kin) {
        va = f32x4{0.f, 0.f, 0.f, 0.f};
        vb = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      *reinterpret_cast<f32x4*>(sA + r * kSP + kq) = va;
      *reinterpret_cast<f32x4*>(sB + r * kSP + kq) = vb;
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  const int steps = (a.K + kBK - 1) / kBK;
  load_tile(0);
  for (int s = 0; s < steps; ++s) {
    __syncthreads();  // every wavefront is done with the previous step's tiles
    store_tile(s * kBK);
    __syncthreads();
    if (s + 1 < steps) load_tile((s + 1) * kBK);  // in flight during the products
#pragma unroll
    for (int g = 0; g < kBK / 8; ++g) {
      f32x4 fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        fa[i] = *reinterpret_cast<const f32x4*>(sA + (wm * 64 + i * 32 + c) * kSP + 8 * g + 4 * hf);
        fb[i] = *reinterpret_cast<const f32x4*>(sB + (wn * 64 + i * 32 + c) * kSP + 8 * g + 4 * hf);
      }
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][t], fb[j][t], acc[i][j], 0, 0, 0);
    }
  }

  // acc[i][j][r]: row m0 + 64 wm + 32 i + 8 (r/4) + 4 hf + r%4, column n0 + 64 wn + 32 j + c
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + wn * 64 + j * 32 + c;
    if (n >= a.N) continue;
    const float bv = a.bias ? a.bias[n] : 0.f;
    const int seg = a.split > 0 ? n / a.split : 0;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
        if (m >= a.M) continue;
        const size_t o = a.split > 0 ? ((size_t)seg * a.M + m) * a.split + (n - seg * a.split)
                                     : (size_t)m * a.N + n;
        float v = acc[i][j][r] + bv;
        if (a.act == 1) v = gelu_tanh_g(v);
        if (a.res) v += a.res[o];
        a.y[o] = v;
      }
  }
}

}  // namespace

// skv_linear's path for calls of more than 64 rows (model_ops.hip). stats
// (may be NULL) holds M * 2 floats for the LayerNorm row statistics.
int gemm_linear(float* y, const float* x, const float* w_t, const float* bias,
                const float* residual, const float* ln_gamma, const float* ln_beta, float ln_eps,
                int M, int N, int K, int activation, int split_cols, float* stats,
                hipStream_t s) {
  const bool ln = ln_gamma != nullptr;
  SKV_REQUIRE((M + kBM - 1) / kBM <= 65535, SKV_E_UNSUPPORTED, "skv_linear: M=%d too large", M);
  if (ln && stats) {
    hipLaunchKernelGGL(k_rowstats, dim3((M + 3) / 4), dim3(256), 0, s, stats, x, M, K, ln_eps);
    const int rc = check_launch("skv_linear");
    if (rc) return rc;
  }
  GemmArgs a{y, x, w_t, bias, residual, ln_gamma, ln_beta, ln ? stats : nullptr, ln_eps,
             M, N, K, activation, split_cols};
  const dim3 grid((N + kBN - 1) / kBN, (M + kBM - 1) / kBM);
  if (ln) hipLaunchKernelGGL(k_gemm<true>, grid, dim3(kThreads), 0, s, a);
  else hipLaunchKernelGGL(k_gemm<false>, grid, dim3(kThreads), 0, s, a);
  return check_launch("skv_linear");
}

}  // namespace skv
