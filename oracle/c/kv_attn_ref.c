/*
 * CPU restatement of the reference's cached decode attention, in fp32.
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/ as a second checker and by
 * bench.py's cpu_baseline leg as the timed CPU baseline. Never linked into
 * the product library.
 *
 * Follows the arithmetic of the reference WGSL kernel
 * create_attention_with_kv_cache_kernel
 * (s-i-e-v-e/llm-experiments simple-llm/src/gpu/gpu_kernels.py:2846-2936):
 *   scale = 1 / sqrt(D)                                    (:2848)
 *   s_t   = (sum_d q[d] * K[t, d], fp32, d ascending) * scale   (:2856-2866)
 *   max   = max(-1e10, s_0 .. s_{len-1})                    (:2872-2888)
 *   e_t   = exp(s_t - max); sum = sum_t e_t                  (:2893-2911)
 *   o[d]  = sum_t (e_t / sum) * V[t, d]                      (:2916-2936)
 * generalised to per-sequence lengths, grouped kv heads and bf16 storage.
 * Parallel over (sequence, head) with OpenMP.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bf16_load(const uint16_t* p, size_t i) {
  uint32_t u = ((uint32_t)p[i]) << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline float elem(const void* base, size_t i, int bf16) {
  return bf16 ? bf16_load((const uint16_t*)base, i) : ((const float*)base)[i];
}

int oracle_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/*
 * q, out: [B, Hq, D] fp32. k, v: [B, T_cap, Hkv, D], fp32 (cache_bf16 = 0)
 * or bf16 bits (cache_bf16 = 1). lens[b] positions are attended.
 * scores: caller scratch of n_threads * T_cap floats.
 */
void oracle_decode_attn(float* out, const float* q, const void* k, const void* v,
                        const int32_t* lens, int B, int Hq, int Hkv, int D, int T_cap,
                        int cache_bf16, float* scores) {
  const int G = Hq / Hkv;
  const float scale = 1.0f / sqrtf((float)D);
#pragma omp parallel for schedule(dynamic, 1)
  for (int bh = 0; bh < B * Hq; ++bh) {
    const int b = bh / Hq, h = bh % Hq, hk = h / G;
#ifdef _OPENMP
    float* s = scores + (size_t)omp_get_thread_num() * T_cap;
#else
    float* s = scores;
#endif
    const float* qv = q + ((size_t)b * Hq + h) * D;
    float* o = out + ((size_t)b * Hq + h) * D;
    int len = lens[b];
    if (len > T_cap) len = T_cap;
    if (len <= 0) {
      for (int d = 0; d < D; ++d) o[d] = 0.f;
      continue;
    }
    float mx = -1e10f;
    for (int t = 0; t < len; ++t) {
      const size_t row = (((size_t)b * T_cap + t) * Hkv + hk) * D;
      float acc = 0.f;
      for (int d = 0; d < D; ++d) acc += qv[d] * elem(k, row + d, cache_bf16);
      s[t] = acc * scale;
      if (s[t] > mx) mx = s[t];
    }
    float sum = 0.f;
    for (int t = 0; t < len; ++t) {
      s[t] = expf(s[t] - mx);
      sum += s[t];
    }
    for (int d = 0; d < D; ++d) o[d] = 0.f;
    for (int t = 0; t < len; ++t) {
      const float w = s[t] / sum;
      const size_t row = (((size_t)b * T_cap + t) * Hkv + hk) * D;
      for (int d = 0; d < D; ++d) o[d] += w * elem(v, row + d, cache_bf16);
    }
  }
}
