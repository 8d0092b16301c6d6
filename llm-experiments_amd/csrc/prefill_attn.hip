// Chunked prefill attention over the cache: MFMA flash attention on gfx950.
//
// Reference behaviour: flash_attention (simple-llm/src/gpu/gpu_pass_forward.py:497-588,
// kernel create_flash_attention_kernel simple-llm/src/gpu/gpu_kernels.py:499-770):
// causal FlashAttention-1, S = Q K^T / sqrt(D), mask kv_pos <= q_pos, online
// softmax, O = sum_t p_t V[t] / l. The reference has no cache offset; here
// query row i of sequence b sits at position start[b] + i and attends cache
// positions [0, start[b] + i], so a chunk is prefilled after an existing
// prefix (the chunk's own K/V must already be appended to the cache).
//
// Design (dense bf16 contraction, MFMA-bound: ~500 flop/byte at C4):
//  * v_mfma_f32_32x32x16_bf16. The kernel computes S^T = K Q^T (K from LDS
//    as operand A, Q held in registers as operand B) so that each lane's
//    accumulator column is one query: the softmax statistics of a query live
//    in one lane pair (lanes l and l^32), and the probabilities P^T come out
//    of the accumulator in exactly the order operand B of the next product
//    O^T += V^T P^T needs (accumulator slot r of rows 8kk..8kk+7 is slot j of
//    k-block kk). Only V needs a transpose, done once per tile while staging
//    it into LDS.
//  * Workgroup = 8 wavefronts of 32 query rows (256 rows). A wavefront fits
//    the 256 registers of two wavefronts per SIMD at D = 128 (148 at D = 64),
//    so two run on each SIMD and the softmax of one overlaps the MFMAs of
//    the other. (With 4 wavefronts of 64 rows, each
//    K/V operand fed two MFMAs, but ~460 registers were live and the
//    compiler shuttled values between AGPRs and VGPRs on every tile: 11%
//    slower, measured on MI355X.) K/V tiles of 64 tokens are double
//    buffered: the global loads of tile t+1 are in flight while tile t is
//    computed. Grouped-query attention folds the G query heads of a kv
//    head into the rows (row = query * G + head), so K/V are read once per
//    group.
//  * Head dims other than 64, 128 and 256 run the same kernel on the head
//    dim padded to DP (32, 64, 128 or 256): K/V tiles go through registers
//    into the same LDS layout, zero-filled past the head dim, and the
//    queries past it are zeros, so QK^T is unchanged and the padded rows of
//    O^T are never stored. At 256 a workgroup has 4 wavefronts (one per
//    SIMD: each holds twice the queries and accumulators) and 128 KB of
//    double-buffered K/V tiles.
//  * Long prefixes are split into n_splits token ranges (split-K, so that
//    about one workgroup runs per CU); partials (m, l, o[D]) are merged by a
//    second pass. The query tiles of one (sequence, kv head, split) are laid
//    out 8 blocks apart so they land on the same XCD together and the second
//    tile's K/V reads hit that XCD's L2. (A merge by the last split of each
//    tile to finish, with the partials written through to memory by
//    device-scope stores, gave the same bits but took the C4 chunk from 568
//    to 621 us on MI355X: 133 KB of write-through stores per workgroup cost
//    more than the 12 us merge pass.)
//  * Rows i >= n_new[b] of the output are written as zeros by the workgroup
//    that owns them (one split) or by the merge pass.
#include <type_traits>

#include "skv_common.h"

namespace skv {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWaves = 8;                   // wavefronts per workgroup up to D = 128
constexpr int kQB = 1;                      // 32-row query blocks per wavefront
constexpr int kBM = kWaves * kQB * 32;      // query rows per workgroup (256)

// Wavefronts per workgroup at kernel head dim D: 8 (two per SIMD) up to 128;
// at 256 a wavefront holds twice the queries and accumulators (~310
// registers), so 4 (one per SIMD, 512 registers each) and 128 query rows.
constexpr int waves_for(int D) { return D > 128 ? 4 : kWaves; }
constexpr int kBN = 64;                     // tokens per K/V tile
constexpr int kXCD = 8;                     // XCDs of an MI355X

struct PrefillArgs {
  const void* q;
  void* out;
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* start;
  const int32_t* n_new;
  int C, Hq, Hkv, T_cap;
  float qscale;  // softmax scale * log2(e)
  int q_dt, out_dt;
  int n_qt;      // query tiles per (sequence, kv head)
  int n_splits;
  int n_groups;  // B * Hkv * n_splits
  float* ws_o;   // [n_splits][B][C][Hq][D]
  float* ws_ml;  // [n_splits][B][C][Hq][2]
  int B;
  int D;         // head dim: the row stride of q, out and the caches
  // skv_append_prefill_attn with a split: workgroup 0 of the attention keeps
  // the fills as the call found them in snap, and the merge pass, which reads
  // them from there, advances the fills in adv (no separate advance launch)
  int32_t* snap;
  int32_t* adv;
};

// K and V tiles live in LDS row-major, [kBN tokens][D] bf16, two stages
// each. The 16-byte chunks of a row are XOR-swizzled, physical chunk =
// chunk ^ key(row), so that both read patterns hit distinct banks of the
// 64-bank (256-byte) LDS: the K operand reads (ds_read_b128) take one chunk
// of 16 consecutive rows, and the V^T reads (ds_read_b64_tr_b16) take 4
// adjacent chunks of 4 consecutive rows per 32 lanes. For D = 128 (16
// chunks per row) key = 4*(row%4) + (row/4)%4 sends the first to 16
// distinct chunks and the second to 16 distinct chunks; for D = 64 (8
// chunks, two rows per bank sweep) key = 4*((row/2)%2) + (row/4)%4 does the
// same. (key = row%16 left the V^T reads 4-way conflicted: measured on
// MI355X, 1e8 conflict cycles per call -> 0, MFMA busy 42% -> 47.5%.)
template <int D>
struct alignas(16) Smem {
  uint16_t k[2][kBN * D];
  uint16_t v[2][kBN * D];
};

template <int D>
__device__ __forceinline__ int swz_key(int row) {
  // D = 256 (32 chunks per row, two bank sweeps) takes the D = 128 key
  if constexpr (D == 128 || D == 256) return 4 * (row & 3) + ((row >> 2) & 3);
  else if constexpr (D == 64) return 4 * ((row >> 1) & 1) + ((row >> 2) & 3);
  else return (row >> 2) & 3;  // D = 32: four chunks per row, four rows per bank sweep
}
template <int D>
__device__ __forceinline__ int swz(int row, int chunk) {  // element offset of a 16-B chunk
  return row * D + ((chunk ^ swz_key<D>(row)) * 8);
}

typedef short i16x4 __attribute__((ext_vector_type(4)));

// 16 bytes from global memory straight into LDS through a buffer descriptor
// (buffer_load_dwordx4 ... lds): lane i writes lds_base + 16 * i with the 16
// bytes at byte offset voff of the buffer, or zeros where voff + 16 passes
// the descriptor's size. lds_base must be the same for every lane. (The
// compiler keeps counting the wavefront's LDS reads in order past these, where
// a pending global_load_lds makes it wait for all of them.)
constexpr int kRsrcW3 = 0x00020000;  // descriptor word 3: raw 32-bit data
__device__ __forceinline__ void buf_dma16(__amdgpu_buffer_rsrc_t rs, uint32_t voff,
                                          const uint16_t* lds_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(lds_base),
                                           16, voff, 0, 0, 0);
}

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives as its slot j
// the element i%4 of the four 16-bit values addressed by lane 4j + i/4.
__device__ __forceinline__ i16x4 lds_read_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(p));
}

// Waits until every memory operation this wavefront issued (including LDS
// DMA writes) has completed.
__device__ __forceinline__ void wait_all_memory() { __builtin_amdgcn_s_waitcnt(0); }

// Four consecutive outputs (16-byte aligned for fp32, 8-byte for bf16).
__device__ __forceinline__ void store4(void* out, size_t i, int dt, const float (&o)[4]) {
  if (dt == SKV_BF16) {
    const uint32_t w0 = (uint32_t)f32_to_bf16(o[0]) | ((uint32_t)f32_to_bf16(o[1]) << 16);
    const uint32_t w1 = (uint32_t)f32_to_bf16(o[2]) | ((uint32_t)f32_to_bf16(o[3]) << 16);
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + i) = make_uint2(w0, w1);
  } else {
    *reinterpret_cast<float4*>(static_cast<float*>(out) + i) = make_float4(o[0], o[1], o[2], o[3]);
  }
}

// LV = 0: D is the real head dim (64 or 128) and tiles move by LDS DMA.
// LV = 8 or 1: D is the padded head dim, a.D the real one; tiles move
// through registers, 16-byte loads (a.D % 8 == 0) or element loads.
template <int D, int G, int LV>
__global__ __launch_bounds__(waves_for(D) * 64, 1) void k_prefill_mfma(PrefillArgs a) {
  constexpr int KB = D / 16;  // k-blocks of the QK^T product
  constexpr int DB = D / 32;  // 32-row d blocks of O^T
  constexpr int W = waves_for(D);
  constexpr int BM = W * kQB * 32;  // query rows of the workgroup
  constexpr bool GEN = LV != 0;
  const int RS = GEN ? a.D : D;  // row stride of q, out and the cache rows
  // LDS stages: register-staged tiles (GEN) share one struct; DMA-staged
  // tiles get one variable per stage, so the compiler sees that a stage's
  // reads cannot alias the DMA landing in the other one and does not make
  // them wait for it.
  __shared__ Smem<GEN ? D : 16> sm;
  __shared__ __attribute__((aligned(16))) uint16_t lds0[GEN ? 8 : 2 * kBN * D];
  __shared__ __attribute__((aligned(16))) uint16_t lds1[GEN ? 8 : 2 * kBN * D];
  auto sk = [&](auto stage) -> uint16_t* {
    constexpr int s_ = decltype(stage)::value;
    if constexpr (GEN) return sm.k[s_];
    else return s_ == 0 ? lds0 : lds1;
  };
  auto sv = [&](auto stage) -> uint16_t* {
    constexpr int s_ = decltype(stage)::value;
    if constexpr (GEN) return sm.v[s_];
    else return (s_ == 0 ? lds0 : lds1) + kBN * D;
  };

  if (a.snap != nullptr && blockIdx.x == 0)
    for (int i = threadIdx.x; i < a.B; i += blockDim.x) a.snap[i] = a.start[i];

  // ---- which (sequence, kv head, split, query tile) this workgroup is ----
  const int w = blockIdx.x;
  const int xcd = w % kXCD, rest = w / kXCD;
  const int qt = rest % a.n_qt;
  const int gi = (rest / a.n_qt) * kXCD + xcd;
  if (gi >= a.n_groups) return;
  const int split = gi % a.n_splits;
  const int bh = gi / a.n_splits;
  const int hk = bh % a.Hkv, b = bh / a.Hkv;

  // Clamped so that no row outside the cache is ever addressed; the host
  // rejects calls whose prefix plus chunk does not fit.
  const int P = min(max(a.start[b], 0), a.T_cap);
  const int n = max(0, min(a.n_new ? min(a.n_new[b], a.C) : a.C, a.T_cap - P));
  const int R = n * G;                 // valid rows of this (b, hk)
  const int row0 = qt * BM;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int lc = lane & 31, g = lane >> 5;

  const int kv_end = P + n;  // tokens [0, kv_end) are in the cache
  int span = (kv_end + a.n_splits - 1) / a.n_splits;
  span = (span + kBN - 1) / kBN * kBN;
  const int s0 = split * span;
  // the last query of this tile bounds the tokens any of its rows attends;
  // a tile past the valid rows has nothing to do
  const int last_row = min(row0 + BM, R) - 1;
  const int s1 = row0 < R ? min(min(s0 + span, kv_end), P + last_row / G + 1) : s0;
  const int first_q = row0 / G;  // smallest query index of the tile

  // ---- queries of this wavefront's two row blocks, as MFMA operand B ----
  bf16x8 qf[kQB][KB];
  int qrow[kQB];
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    const int r = row0 + (wave * kQB + qb) * 32 + lc;
    qrow[qb] = r;
    const bool ok = r < R;
    const int i = r / G, h = hk * G + r % G;
    const size_t qoff = (((size_t)b * a.C + i) * a.Hq + h) * RS;
    const size_t qsafe = ok ? qoff : 0;  // rows past the chunk read row 0 and are zeroed
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      float v[8];
      if constexpr (GEN) {  // element loads at clamped offsets, zeros past the head dim
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int e = kb * 16 + g * 8 + j;
          const float x = load_elem(a.q, e < RS ? qsafe + e : 0, a.q_dt);
          v[j] = e < RS ? x : 0.f;
        }
      } else {
        load8_f32(a.q, qsafe + kb * 16 + g * 8, a.q_dt, v);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) qf[qb][kb][j] = (__bf16)(ok ? v[j] : 0.f);
    }
  }

  f32x16 o[kQB][DB];
  float m[kQB], l[kQB];
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    m[qb] = -INFINITY;
    l[qb] = 0.f;
#pragma unroll
    for (int db = 0; db < DB; ++db) o[qb][db] = f32x16{};
  }

  const size_t row_stride = (size_t)a.Hkv * RS;  // elements between consecutive tokens
  const uint16_t* kbase = a.k + ((size_t)b * a.T_cap * a.Hkv + hk) * RS;
  const uint16_t* vbase = a.v + ((size_t)b * a.T_cap * a.Hkv + hk) * RS;

  // Tiles go from HBM straight into LDS (buffer_load_dwordx4 ... lds: each
  // lane moves 16 bytes, a wavefront fills 1 KB of LDS in lane order), so no
  // registers are spent on staging. A lane picks the global chunk that the
  // swizzled layout stores at its LDS position. Each tile's descriptor starts
  // at its first row and covers only the rows below kv_end, so rows past it
  // read zeros (masked later) and nothing outside the cache is addressed; the
  // tile after the last one is fetched too and never read. (With the DMA as
  // global_load_lds the compiler waited for every pending LDS read before
  // each MFMA operand, as a pending global access that writes LDS made it
  // stop counting them in order: 552.2 -> 531.9 us per C4 chunk, same bits.)
  constexpr int RPK = 1024 / (D * 2);          // token rows per 1 KB
  constexpr int KPT = kBN * D * 2 / 1024;      // 1 KB pieces per tile and tensor
  static_assert(GEN || KPT % W == 0, "tile pieces must split over the wavefronts");
  // Register-staged tiles (GEN): 16-byte chunk c of a tile is token row
  // c / (D/8), logical chunk c % (D/8), at the same swizzled LDS position as
  // the DMA form; chunks past the head dim are zeros.
  constexpr int NCH = kBN * D / 8;                             // chunks per tile and tensor
  constexpr int CPT = (NCH + W * 64 - 1) / (W * 64);  // chunks per thread
  uint4 rk[GEN ? CPT : 1], rv[GEN ? CPT : 1];
  auto reg_tile_load = [&](int T0) {
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int c = min(tid + u * W * 64, NCH - 1);  // threads past NCH repeat the last chunk
      const int row = c / (D / 8), lch = c % (D / 8);
      const size_t rofs = (size_t)min(T0 + row, kv_end - 1) * row_stride;
      if constexpr (LV == 8) {
        const bool ok = lch * 8 < RS;  // RS % 8 == 0: the chunk is wholly inside or past D
        const uint4 zk = *reinterpret_cast<const uint4*>(kbase + rofs + (ok ? lch * 8 : 0));
        const uint4 zv = *reinterpret_cast<const uint4*>(vbase + rofs + (ok ? lch * 8 : 0));
        rk[u] = ok ? zk : make_uint4(0, 0, 0, 0);
        rv[u] = ok ? zv : make_uint4(0, 0, 0, 0);
      } else {
        uint32_t wk[4], wv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int e0 = lch * 8 + 2 * j;
          const uint32_t k0 = kbase[rofs + (e0 < RS ? e0 : 0)];
          const uint32_t k1 = kbase[rofs + (e0 + 1 < RS ? e0 + 1 : 0)];
          const uint32_t v0 = vbase[rofs + (e0 < RS ? e0 : 0)];
          const uint32_t v1 = vbase[rofs + (e0 + 1 < RS ? e0 + 1 : 0)];
          wk[j] = (e0 < RS ? k0 : 0u) | ((e0 + 1 < RS ? k1 : 0u) << 16);
          wv[j] = (e0 < RS ? v0 : 0u) | ((e0 + 1 < RS ? v1 : 0u) << 16);
        }
        rk[u] = make_uint4(wk[0], wk[1], wk[2], wk[3]);
        rv[u] = make_uint4(wv[0], wv[1], wv[2], wv[3]);
      }
    }
  };
  auto reg_tile_store = [&](int ST) {
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int c = tid + u * W * 64;
      if (c >= NCH) continue;
      const int row = c / (D / 8), lch = c % (D / 8);
      *reinterpret_cast<uint4*>(&sm.k[ST][swz<D>(row, lch)]) = rk[u];
      *reinterpret_cast<uint4*>(&sm.v[ST][swz<D>(row, lch)]) = rv[u];
    }
  };
  // Per lane, the byte offset of its 16-byte chunk within a tile (the same
  // for every tile): token row piece * RPK + lane / (D / 8), swizzled chunk.
  uint32_t dma_off[GEN ? 1 : KPT / W];
  if constexpr (!GEN) {
#pragma unroll
    for (int c = 0; c < KPT / W; ++c) {
      const int piece = wave * (KPT / W) + c;
      const int row = piece * RPK + lane / (D / 8);
      const int lch = (lane % (D / 8)) ^ swz_key<D>(row);
      dma_off[c] = (uint32_t)(row * row_stride + lch * 8) * 2u;
    }
  }
#define SKV_DMA_TILE(T0, ST)                                                                 \
  if constexpr (!GEN) {                                                                      \
    /* a buffer over the tile's rows that exist: rows past kv_end read zeros */             \
    const int rows_ = max(0, min(kv_end - (T0), kBN));                                       \
    const int nrec_ = rows_ > 0 ? (int)(((rows_ - 1) * row_stride + D) * 2) : 0;           \
    const size_t base_ = (size_t)max(min((T0), kv_end - 1), 0) * row_stride;               \
    const __amdgpu_buffer_rsrc_t rk_ =                                                       \
        __builtin_amdgcn_make_buffer_rsrc((void*)(kbase + base_), (short)0, nrec_, kRsrcW3);  \
    const __amdgpu_buffer_rsrc_t rv_ =                                                       \
        __builtin_amdgcn_make_buffer_rsrc((void*)(vbase + base_), (short)0, nrec_, kRsrcW3);  \
    _Pragma("unroll") for (int c = 0; c < KPT / W; ++c) {                                    \
      const int piece = wave * (KPT / W) + c;                                                \
      buf_dma16(rk_, dma_off[c], sk(std::integral_constant<int, (ST)>{}) + piece * 512);     \
      buf_dma16(rv_, dma_off[c], sv(std::integral_constant<int, (ST)>{}) + piece * 512);     \
    }                                                                                        \
  }

  const int n_tiles = s1 > s0 ? (s1 - s0 + kBN - 1) / kBN : 0;
  if constexpr (GEN) {
    if (n_tiles > 0) {
      reg_tile_load(s0);
      reg_tile_store(0);
    }
  } else {
    if (n_tiles > 0) SKV_DMA_TILE(s0, 0);
  }
  wait_all_memory();
  __syncthreads();

  // One tile; the LDS stage is a compile-time constant (the loop below runs
  // stage 0 and stage 1 in turn), so every LDS address is a loop-invariant
  // per-lane offset plus an immediate. With the stage as a runtime value the
  // compiler recomputed ~70 addresses per tile with integer adds, a third of
  // the loop's VALU instructions.
  auto tile = [&](auto stage, int it) {
    constexpr int st = decltype(stage)::value;
    const int t0 = s0 + it * kBN;
    // the next tile: DMA into the other stage, or (GEN) loads into registers
    // now and their LDS stores after this tile's products
    // (At D = 256 the registers of a staged tile are not free during the
    // products: its loads wait until after them, see the end of the tile.)
    if constexpr (GEN && D <= 128) reg_tile_load(t0 + kBN);
    else if constexpr (!GEN) SKV_DMA_TILE(t0 + kBN, st ^ 1);

    // S^T for the whole 64-token tile first (two independent accumulator
    // chains per query block), then one online-softmax update, then PV.
    const bool need_mask = (t0 + kBN > s1) || (t0 + kBN - 1 > P + first_q);
    f32x16 sc[2][kQB];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
      for (int qb = 0; qb < kQB; ++qb) sc[tb][qb] = f32x16{};
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) {
        const bf16x8 ka =
            *reinterpret_cast<const bf16x8*>(sk(stage) + swz<D>(tb * 32 + lc, kb * 2 + g));
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb)
          sc[tb][qb] =
              __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qf[qb][kb], sc[tb][qb], 0, 0, 0);
      }
    // Accumulator slot r of half tb holds token t0 + tb*32 + (r/4)*8 + 4g + r%4.
    if (need_mask) {
#pragma unroll
      for (int qb = 0; qb < kQB; ++qb) {
        const int qpos = P + qrow[qb] / G;  // this lane's query position
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int t = t0 + tb * 32 + (r >> 2) * 8 + g * 4 + (r & 3);
            sc[tb][qb][r] = (t >= s1 || t > qpos) ? -INFINITY : sc[tb][qb][r];
          }
      }
    }
    // ---- online softmax; P^T as operand B of the PV product ----
    bf16x8 pf[kQB][4];  // [qb][tb * 2 + kk]
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
      float tmax = sc[0][qb][0];
#pragma unroll
      for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, sc[tb][qb][r]);
      tmax = xor32_max(tmax);  // lanes l and l ^ 32 hold the same query
      // Lazy rescaling: the running max m only moves when the tile's max
      // exceeds it by more than 8 (log2 units), so probabilities stay
      // <= 2^8 (exact in fp32, in range for bf16) and O, l are rescaled
      // on a few tiles instead of every one. O and l always refer to the
      // same m.
      const float tm = tmax * a.qscale;
      const bool upd = tm > m[qb] + 8.f;  // also true on the first finite tile
      if (__ballot(upd) != 0ull) {        // wave-uniform branch
        const float alpha = upd ? fast_exp2(m[qb] - tm) : 1.f;  // m = -inf: 0
        if (upd) m[qb] = tm;
        l[qb] *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db) o[qb][db] *= alpha;
      }
      const float m_use = m[qb] == -INFINITY ? 0.f : m[qb];  // fully masked so far
      float ls = 0.f;
#pragma unroll
      for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float p = fast_exp2(fmaf(sc[tb][qb][kk * 8 + j], a.qscale, -m_use));
            ls += p;
            pf[qb][tb * 2 + kk][j] = (__bf16)p;
          }
      l[qb] += ls;
    }
    // ---- O^T += V^T P^T ----
    // Operand A of k-block kk needs, in lane (d = db*32 + lc, g), slot j =
    // V[tb*32 + 16kk + 4g + j][d] for j < 4 and V[... + 8 + 4g + j - 4][d]
    // for j >= 4 (the token order of pf). ds_read_b64_tr_b16 gives lane i
    // of a 16-lane group the element i%4 of the 8 bytes addressed by lane
    // 4j + i/4 as its slot j, so lane L of group gr addresses token
    // T + 4g + L/4, elements d0 + 4(L%4) .. +3 with d0 = db*32 + (gr%2)*16.
    {
      const int gr = lane >> 4, L = lane & 15;
      const int dq = (gr & 1) * 16 + 4 * (L & 3);  // d offset within the 32-row block
      // kk outside db: consecutive MFMAs accumulate into different O blocks
      // (each block still takes its four k-blocks in the same order)
#pragma unroll
      for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            const int d = db * 32 + dq;
            const int r0 = tb * 32 + kk * 16 + 4 * g + (L >> 2);
            const int r1 = r0 + 8;
            const uint16_t* p0 = sv(stage) + swz<D>(r0, d >> 3) + (d & 7);
            const uint16_t* p1 = sv(stage) + swz<D>(r1, d >> 3) + (d & 7);
            const i16x4 lo = lds_read_tr16(p0);
            const i16x4 hi = lds_read_tr16(p1);
            const bf16x8 va = __builtin_bit_cast(
                bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
            for (int qb = 0; qb < kQB; ++qb)
              o[qb][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pf[qb][tb * 2 + kk],
                                                                   o[qb][db], 0, 0, 0);
          }
    }

    if constexpr (GEN && D > 128) reg_tile_load(t0 + kBN);
    if constexpr (GEN) reg_tile_store(st ^ 1);
    // the next tile's DMA has landed in LDS before anyone reads it
    wait_all_memory();
    __syncthreads();
  };
  for (int it = 0; it < n_tiles; it += 2) {
    tile(std::integral_constant<int, 0>{}, it);
    if (it + 1 < n_tiles) tile(std::integral_constant<int, 1>{}, it + 1);
  }
#undef SKV_DMA_TILE

  // ---- epilogue: this lane holds query column lc of each row block; the
  // accumulator slot r of d block db is d = db*32 + (r/4)*8 + 4g + r%4 ----
  const int CG = a.C * G;  // output rows of this (b, hk): query i, head h -> i * G + h % G
  float lt[kQB];
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) lt[qb] = xor32_sum(l[qb]);
  // Row r's output from its normalised values v(db, r4, e), or zeros for a
  // row past the sequence's new tokens; rows past the chunk are not stored.
  auto store_row = [&](int r, auto&& v) {
    if (r >= CG) return;
    const int i = r / G, h = hk * G + r % G;
    const size_t orow = ((size_t)b * a.C + i) * a.Hq + h;
    const bool valid = r < R;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d0 = db * 32 + r4 * 8 + g * 4;
        float x[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = valid ? v(db, r4, e) : 0.f;
        if constexpr (GEN) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (d0 + e < RS) store_elem(a.out, orow * RS + d0 + e, a.out_dt, x[e]);
        } else {
          store4(a.out, orow * D + d0, a.out_dt, x);
        }
      }
  };
  if (a.n_splits == 1) {
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
      const float inv = 1.f / lt[qb];
      store_row(qrow[qb], [&](int db, int r4, int e) { return o[qb][db][r4 * 4 + e] * inv; });
    }
    return;
  }
  // n_splits > 1: this split's partial of every valid row, for the merge pass
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    const int r = qrow[qb];
    if (r >= R) continue;
    const int i = r / G, h = hk * G + r % G;
    const size_t prow = (size_t)split * a.B * a.C * a.Hq + ((size_t)b * a.C + i) * a.Hq + h;
    float* dst = a.ws_o + prow * D;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        float4 x;
        x.x = o[qb][db][r4 * 4 + 0];
        x.y = o[qb][db][r4 * 4 + 1];
        x.z = o[qb][db][r4 * 4 + 2];
        x.w = o[qb][db][r4 * 4 + 3];
        *reinterpret_cast<float4*>(dst + db * 32 + r4 * 8 + g * 4) = x;
      }
    if (g == 0) {
      a.ws_ml[prow * 2 + 0] = m[qb];
      a.ws_ml[prow * 2 + 1] = lt[qb];
    }
  }
}

constexpr int kMergeBatch = 4;  // splits whose partials the merge loads in one round trip

// Merge of the split partials, grid (tiles of C * Hq * D/4 threads, B): one
// thread per 4 consecutive d of a row, 16-byte partial loads, 32-bit index
// arithmetic. (One thread per element with 64-bit divisions took 31 us on
// C4's 55 MB, 1.7 TB/s, measured on MI355X.) Rows i >= n_new[b] are zeros.
// Splits that saw no token of a row (m = -inf, l = 0) drop out. The partials
// have the kernel's (padded) row stride D; GEN: outputs have the real head
// dim a.D, stored element by element.
template <int D, bool GEN>
__global__ __launch_bounds__(256) void k_prefill_merge(PrefillArgs a) {
  constexpr int V = D / 4;  // threads per row
  const int b = blockIdx.y;
  const int g = blockIdx.x * 256 + threadIdx.x;
  if (g >= a.C * a.Hq * V) return;
  const int rb = g / V, d = (g % V) * 4;  // row within the sequence: i * Hq + h
  const int i = rb / a.Hq;
  const size_t rows = (size_t)a.B * a.C * a.Hq;
  const size_t row = (size_t)b * a.C * a.Hq + rb;
  // the fill as the call found it (from the snapshot when this pass also
  // advances it: nothing here reads the fills themselves then)
  const int P0 = a.snap != nullptr ? a.snap[b] : a.start[b];
  if (a.adv != nullptr && blockIdx.x == 0 && threadIdx.x == 0)
    a.adv[b] = min(P0 + (a.n_new ? a.n_new[b] : a.C), a.T_cap);  // skv_advance's rule
  const int P = min(max(P0, 0), a.T_cap);
  const int n = max(0, min(a.n_new ? min(a.n_new[b], a.C) : a.C, a.T_cap - P));
  float o[4] = {0.f, 0.f, 0.f, 0.f};
  // One split's weighted partial into (L, o), in split order.
  auto add = [&](float2 ml, float4 x, float M, float& L) {
    if (ml.x == -INFINITY) return;
    const float wgt = fast_exp2(ml.x - M);
    L = fmaf(wgt, ml.y, L);
    o[0] = fmaf(wgt, x.x, o[0]);
    o[1] = fmaf(wgt, x.y, o[1]);
    o[2] = fmaf(wgt, x.z, o[2]);
    o[3] = fmaf(wgt, x.w, o[3]);
  };
  if (i < n) {
    float M = -INFINITY, L = 0.f;
    if (a.n_splits <= kMergeBatch) {
      // every split's (m, l) and o loaded together: one memory round trip
      float2 ml[kMergeBatch];
      float4 x[kMergeBatch];
#pragma unroll
      for (int s = 0; s < kMergeBatch; ++s) {
        const size_t pr = (size_t)min(s, a.n_splits - 1) * rows + row;
        ml[s] = *reinterpret_cast<const float2*>(a.ws_ml + pr * 2);
        x[s] = *reinterpret_cast<const float4*>(a.ws_o + pr * D + d);
      }
#pragma unroll
      for (int s = 0; s < kMergeBatch; ++s)
        if (s < a.n_splits) M = fmaxf(M, ml[s].x);
#pragma unroll
      for (int s = 0; s < kMergeBatch; ++s)
        if (s < a.n_splits) add(ml[s], x[s], M, L);
    } else {
      for (int s = 0; s < a.n_splits; ++s) M = fmaxf(M, a.ws_ml[(s * rows + row) * 2]);
      for (int s = 0; s < a.n_splits; ++s) {
        const size_t pr = s * rows + row;
        add(*reinterpret_cast<const float2*>(a.ws_ml + pr * 2),
            *reinterpret_cast<const float4*>(a.ws_o + pr * D + d), M, L);
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = o[e] / L;
  }
  if constexpr (GEN) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (d + e < a.D) store_elem(a.out, row * a.D + d + e, a.out_dt, o[e]);
  } else {
    store4(a.out, row * D + d, a.out_dt, o);
  }
}

// Query tiles of a (sequence, kv head) at kernel head dim DK (the plan,
// which does not know the head dim, counts them at DK = 128).
int n_query_tiles(int C, int G, int DK = 128) {
  const int bm = waves_for(DK) * kQB * 32;
  return (C * G + bm - 1) / bm;
}

// Head dim the bf16 kernel runs at: 64, 128 and 256 as they are, others
// padded to the next of 32, 64, 128, 256.
int kernel_dim(int D) {
  if (D == 64 || D == 128 || D >= 256) return D;
  return D <= 32 ? 32 : D <= 64 ? 64 : D <= 128 ? 128 : 256;
}

bool dt_ok(int dt) { return dt == SKV_F32 || dt == SKV_BF16; }

}  // namespace
}  // namespace skv

using namespace skv;

namespace {
size_t prefill_part_bytes(int B, int C, int H_q, int D, int n_splits) {
  return (size_t)n_splits * B * C * H_q * (size_t)(kernel_dim(D) + 2) * sizeof(float);
}
}  // namespace

extern "C" int skv_prefill_plan(int B, int C, int H_q, int H_kv, int max_kv_end, int* n_splits) {
  SKV_REQUIRE(n_splits, SKV_E_INVALID, "skv_prefill_plan: null output");
  SKV_REQUIRE(B > 0 && C > 0 && H_q > 0 && H_kv > 0 && max_kv_end > 0 && H_q % H_kv == 0,
              SKV_E_INVALID, "skv_prefill_plan: bad dims (B=%d C=%d H_q=%d H_kv=%d len=%d)", B,
              C, H_q, H_kv, max_kv_end);
  // About one workgroup per CU (256 on MI355X), and splits of at least four
  // 64-token tiles.
  const long wg = (long)B * H_kv * n_query_tiles(C, H_q / H_kv);
  long ns = (256 + wg - 1) / wg;
  const long max_ns = (max_kv_end + 4 * kBN - 1) / (4 * kBN);
  if (ns > max_ns) ns = max_ns;
  if (ns > 32) ns = 32;
  if (ns < 1) ns = 1;
  *n_splits = (int)ns;
  return SKV_OK;
}

extern "C" size_t skv_prefill_workspace_bytes(int B, int C, int H_q, int D, int n_splits) {
  if (B <= 0 || C <= 0 || H_q <= 0 || D <= 0 || n_splits <= 1) return 0;
  // partials at the kernel's (padded) head dim, then the fills' snapshot of
  // skv_append_prefill_attn (B int32, 16-byte padded)
  return prefill_part_bytes(B, C, H_q, D, n_splits) + ((size_t)B * sizeof(int32_t) + 15) / 16 * 16;
}

namespace {

// skv_prefill_attn's checks and launches. adv (split bf16 path only): the
// merge pass advances these fills (skv_advance's rule) from the snapshot at
// the end of ws. launch = false: the checks alone, nothing launched.
int prefill_attn_impl(void* out, const void* q, const void* k_cache, const void* v_cache,
                      const int32_t* start, const int32_t* n_new, int B, int C, int H_q,
                      int H_kv, int D, int T_cap, float scale, int n_splits, void* ws,
                      size_t ws_bytes, int cache_dt, int q_dt, int out_dt, skv_stream_t stream,
                      const char* fn, int32_t* adv, bool launch) {
  SKV_REQUIRE(out && q && k_cache && v_cache && start, SKV_E_INVALID, "%s: null pointer argument",
              fn);
  SKV_REQUIRE(B > 0 && C > 0 && H_q > 0 && H_kv > 0 && T_cap > 0, SKV_E_INVALID,
              "%s: dims must be > 0", fn);
  SKV_REQUIRE(H_q % H_kv == 0, SKV_E_INVALID, "%s: H_q=%d not a multiple of H_kv=%d", fn, H_q,
              H_kv);
  SKV_REQUIRE(dt_ok(cache_dt) && dt_ok(q_dt) && dt_ok(out_dt), SKV_E_INVALID, "%s: bad dtype",
              fn);
  SKV_REQUIRE(scale > 0.f, SKV_E_INVALID, "%s: scale must be > 0", fn);
  if (cache_dt == SKV_F32) {  // fp32 cache: the fp32 MFMA path, no split
    SKV_REQUIRE(q_dt == SKV_F32 && out_dt == SKV_F32, SKV_E_UNSUPPORTED,
                "%s: an fp32 cache takes fp32 q and out", fn);
    if (!launch) {  // attn_fwd_f32's own checks (128 queries a workgroup there)
      SKV_REQUIRE(D >= 1 && D <= 256, SKV_E_UNSUPPORTED, "%s: head_dim %d (supported: 1 to 256)",
                  fn, D);
      SKV_REQUIRE((((uintptr_t)out | (uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) &
                   15) == 0,
                  SKV_E_INVALID, "%s: q, k, v and out must be 16-byte aligned", fn);
      SKV_REQUIRE((long)((C + 127) / 128) * B * H_q < (1L << 31), SKV_E_UNSUPPORTED,
                  "%s: grid too large", fn);
      return SKV_OK;
    }
    return attn_fwd_f32(static_cast<float*>(out), nullptr, nullptr, static_cast<const float*>(q),
                        static_cast<const float*>(k_cache), static_cast<const float*>(v_cache),
                        start, n_new, B, C, H_q, H_kv, D, T_cap, scale, (hipStream_t)stream, fn);
  }
  SKV_REQUIRE(D >= 1 && D <= 256, SKV_E_UNSUPPORTED, "%s: head_dim %d (supported: 1 to 256)",
              fn, D);
  SKV_REQUIRE((((uintptr_t)out | (uintptr_t)q | (uintptr_t)ws | (uintptr_t)k_cache |
                (uintptr_t)v_cache) & 15) == 0,
              SKV_E_INVALID, "%s: out, q, the caches and ws must be 16-byte aligned", fn);
  const int DK = kernel_dim(D);  // the kernel's (padded) head dim
  SKV_REQUIRE((size_t)C * H_q * D < (1u << 31), SKV_E_UNSUPPORTED, "%s: chunk too large", fn);
  // a K/V tile's buffer descriptor spans kBN cache rows of H_kv * D elements
  // (32-bit byte counts)
  SKV_REQUIRE((long)H_kv * D * kBN * 2 < (1L << 31), SKV_E_UNSUPPORTED,
              "%s: cache rows too wide (H_kv * head_dim = %ld)", fn, (long)H_kv * D);
  const int G = H_q / H_kv;
  SKV_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, SKV_E_UNSUPPORTED,
              "%s: no kernel for G=%d", fn, G);
  SKV_REQUIRE(n_splits >= 1 && n_splits <= 32, SKV_E_INVALID, "%s: n_splits=%d out of range", fn,
              n_splits);
  if (n_splits > 1) {
    const size_t need = skv_prefill_workspace_bytes(B, C, H_q, D, n_splits);
    SKV_REQUIRE(ws && ws_bytes >= need, SKV_E_WORKSPACE, "%s: workspace %zu bytes < %zu required",
                fn, ws_bytes, need);
  }
  PrefillArgs a;
  a.snap = nullptr;
  a.adv = nullptr;
  if (adv != nullptr && n_splits > 1) {
    a.adv = adv;
    a.snap = reinterpret_cast<int32_t*>(static_cast<char*>(ws) +
                                        prefill_part_bytes(B, C, H_q, D, n_splits));
  }
  a.q = q; a.out = out;
  a.k = static_cast<const uint16_t*>(k_cache);
  a.v = static_cast<const uint16_t*>(v_cache);
  a.start = start; a.n_new = n_new;
  a.C = C; a.Hq = H_q; a.Hkv = H_kv; a.T_cap = T_cap;
  a.qscale = scale * LOG2E;
  a.q_dt = q_dt; a.out_dt = out_dt;
  a.n_qt = n_query_tiles(C, G, DK);
  a.n_splits = n_splits;
  a.n_groups = B * H_kv * n_splits;
  a.B = B;
  a.D = D;
  a.ws_o = static_cast<float*>(ws);
  a.ws_ml = n_splits > 1 ? a.ws_o + (size_t)n_splits * B * C * H_q * DK : nullptr;
  const long blocks = (long)((a.n_groups + kXCD - 1) / kXCD) * kXCD * a.n_qt;
  SKV_REQUIRE(blocks < (1L << 31), SKV_E_UNSUPPORTED, "%s: grid too large", fn);
  if (!launch) return SKV_OK;
  hipStream_t s = (hipStream_t)stream;
  // LV: 0 = LDS DMA at the exact head dim; 8 = 16-byte register loads; 1 = element loads
  const int LV = DK == D ? 0 : (D % 8 == 0 ? 8 : 1);
#define SKV_PF(DD, GG, LL)                                                                    \
  if (DK == DD && G == GG && LV == LL)                                                        \
    hipLaunchKernelGGL((k_prefill_mfma<DD, GG, LL>), dim3((unsigned)blocks),                  \
                       dim3(waves_for(DD) * 64), 0, s, a);
#define SKV_PF4(DD, LL) SKV_PF(DD, 1, LL) SKV_PF(DD, 2, LL) SKV_PF(DD, 4, LL) SKV_PF(DD, 8, LL)
  SKV_PF4(64, 0) SKV_PF4(128, 0) SKV_PF4(256, 0)
  SKV_PF4(32, 8) SKV_PF4(32, 1) SKV_PF4(64, 8) SKV_PF4(64, 1) SKV_PF4(128, 8) SKV_PF4(128, 1)
  SKV_PF4(256, 8) SKV_PF4(256, 1)
#undef SKV_PF4
#undef SKV_PF
  int rc = check_launch(fn);
  if (rc) return rc;
  if (n_splits > 1) {
    const dim3 mgrid((unsigned)(((size_t)C * H_q * (DK / 4) + 255) / 256), (unsigned)B);
    if (LV == 0 && D == 64) hipLaunchKernelGGL((k_prefill_merge<64, false>), mgrid, dim3(256), 0, s, a);
    else if (LV == 0 && D == 128) hipLaunchKernelGGL((k_prefill_merge<128, false>), mgrid, dim3(256), 0, s, a);
    else if (LV == 0) hipLaunchKernelGGL((k_prefill_merge<256, false>), mgrid, dim3(256), 0, s, a);
    else if (DK == 32) hipLaunchKernelGGL((k_prefill_merge<32, true>), mgrid, dim3(256), 0, s, a);
    else if (DK == 64) hipLaunchKernelGGL((k_prefill_merge<64, true>), mgrid, dim3(256), 0, s, a);
    else if (DK == 128) hipLaunchKernelGGL((k_prefill_merge<128, true>), mgrid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((k_prefill_merge<256, true>), mgrid, dim3(256), 0, s, a);
  }
  return check_launch(fn);
}

}  // namespace

extern "C" int skv_prefill_attn(void* out, const void* q, const void* k_cache,
                                const void* v_cache, const int32_t* start, const int32_t* n_new,
                                int B, int C, int H_q, int H_kv, int D, int T_cap, float scale,
                                int n_splits, void* ws, size_t ws_bytes, int cache_dt, int q_dt,
                                int out_dt, skv_stream_t stream) {
  return prefill_attn_impl(out, q, k_cache, v_cache, start, n_new, B, C, H_q, H_kv, D, T_cap,
                           scale, n_splits, ws, ws_bytes, cache_dt, q_dt, out_dt, stream,
                           "skv_prefill_attn", nullptr, true);
}

extern "C" int skv_append_prefill_attn(void* out, const void* q, void* k_cache, void* v_cache,
                                       const void* k_new, const void* v_new, int32_t* lens,
                                       const int32_t* n_new, int B, int C, int H_q, int H_kv,
                                       int D, int T_cap, float scale, int n_splits, void* ws,
                                       size_t ws_bytes, int cache_dt, int in_dt, int q_dt,
                                       int out_dt, skv_stream_t stream) {
  const char* fn = "skv_append_prefill_attn";
  // every check of the attention first, so that a rejected call changes nothing
  int rc = prefill_attn_impl(out, q, k_cache, v_cache, lens, n_new, B, C, H_q, H_kv, D, T_cap,
                             scale, n_splits, ws, ws_bytes, cache_dt, q_dt, out_dt, stream, fn,
                             lens, false);
  if (rc) return rc;
  rc = skv_append_chunk(k_cache, v_cache, k_new, v_new, lens, n_new, B, C, H_kv, D, T_cap,
                        cache_dt, in_dt, stream);
  if (rc) return rc;
  rc = prefill_attn_impl(out, q, k_cache, v_cache, lens, n_new, B, C, H_q, H_kv, D, T_cap, scale,
                         n_splits, ws, ws_bytes, cache_dt, q_dt, out_dt, stream, fn, lens, true);
  if (rc) return rc;
  // the split bf16 path's merge pass has advanced the fills; the others advance here
  if (cache_dt == SKV_BF16 && n_splits > 1) return SKV_OK;
  return skv_advance(lens, n_new, C, B, T_cap, stream);
}
