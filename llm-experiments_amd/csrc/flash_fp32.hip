// Causal FlashAttention in fp32 on gfx950: the forward with its row
// statistics (skv_flash_fwd, also the fp32-cache path of skv_prefill_attn)
// and the backward (skv_flash_bwd), on v_mfma_f32_32x32x2_f32 (fp32
// products, fp32 accumulation). The notes below describe the backward; the
// forward reuses its tiling.
//
// Reference: simple-llm/src/gpu/gpu_kernels.py:2038-2455 (stage 1, one pass
// per Q block writing partial dK/dV into a workspace; stage 2, their sum) and
// the dispatcher gpu/gpu_pass_backward.py:445-580. Per (batch b, head h), with
// S = scale * Q K^T, masked to key <= query:
//   P  = exp(S - M) / L          M, L: the forward's row statistics
//   Dl = rowsum(dO * O)          O: the forward's output
//   dP = dO V^T,  dS = P * (dP - Dl)
//   dQ = scale * dS K,  dK = scale * dS^T Q,  dV = P^T dO
//
// Design: two kernels, no atomics and every sum in a fixed order, so a call
// is bitwise reproducible:
//   k_fbwd_dq   one workgroup per (128 queries, b, h). Per 32-key piece:
//               S^T = K Q^T and dP^T = V dO^T, then dQ^T += K^T dS^T. It
//               also writes Dl for the second kernel.
//   k_fbwd_dkv  one workgroup per (128 keys, b, h). Per 32-query piece:
//               S = Q K^T and dP = dO V^T, then dV += P^T dO, dK += dS^T Q.
// Each of the 4 waves owns 32 rows. Its row operands (Q and dO, or K and V)
// stay in registers for the whole call (up to a head dim of 64, k_fbwd_dkv
// keeps V in LDS instead); the other side is staged through LDS 64 rows at a
// time, the next rows' global loads issued a step ahead, into registers, or,
// where the kernel runs more wavefronts per SIMD (D <= 64: two for
// k_fbwd_dkv, three for k_fbwd_dq and the forward), at the top of each step.
// Work past the causal diagonal is skipped per wave.
//
// v_mfma_f32_32x32x2_f32 lane layout (lane l, c = l % 32, hf = l / 32):
//   A (32 x 2): A[c][hf]   B (2 x 32): B[hf][c]
//   C (32 x 32), register r: row 8*(r/4) + 4*hf + r%4, column c.
// The k index of a product is free to permute as long as A and B agree:
// step (g, t) of a D-long dot product takes d = 8g + 4hf + t in half hf, so
// each lane reads 4 consecutive d with one 16-byte load per 4 steps. A
// C-layout tile is then directly the A or B operand of the next product,
// k-step (q, t) taking row 8q + 4hf + t.
#include "skv_common.h"

namespace skv {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kRows = 32 * kWaves;  // rows (queries or keys) of one workgroup
constexpr int kCols = 64;           // rows of the other side staged per step

struct FbwdArgs {
  const float* q;
  const float* k;
  const float* v;
  const float* o;
  const float* dout;
  const float* L;
  const float* M;
  float* dq;
  float* dk;
  float* dv;
  float* delta;  // [B, N, H] row deltas Dl, written by k_fbwd_dq (or k_fbwd_delta)
  float* ds;     // dS in 32 x 32 tiles (see ds_tile), written by k_fbwd_dkv<.., true> for k_fbwd_dq_ds
  int N, H, BH, n_blocks;
  int D;  // head dim (the padded size is the kernel's template D)
  float scale, sl2;  // scale and scale * log2(e)
};

__device__ __forceinline__ f32x16 mfma(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// 2^x on v_exp_f32 (results below 2^-126 flush toward 0, which no
// probability here needs).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Element offset of row n of head h in batch b of a [B, N, H, D] tensor.
__device__ __forceinline__ size_t row_off(int b, int n, int N, int H, int h, int D) {
  return ((size_t)(b * N + n) * H + h) * D;
}

// Head dims: the kernels run on the head dim padded to DP, a multiple of 16
// (two 8-element k groups per row fragment, whole float4 LDS stores). MODE
// 0: D == DP (16, 32, 64, 128), 16-byte vectors throughout; MODE 1: D < DP
// with D % 4 == 0 (float4 loads, groups past D read as zeros); MODE 2: any
// other D (element loads). Padded elements are zeros in every operand that
// is contracted over d, and the output rows they produce are never stored,
// so results equal the unpadded computation.
// Four consecutive elements c..c+3 of a row with D elements, zeros past D.
template <int MODE>
__device__ __forceinline__ f32x4 load4m(const float* row, int c, int D) {
  if constexpr (MODE == 0) {
    return *reinterpret_cast<const f32x4*>(row + c);
  } else if constexpr (MODE == 1) {
    const bool ok = c < D;  // D % 4 == 0: the group lies wholly inside or past D
    const f32x4 x = *reinterpret_cast<const f32x4*>(row + (ok ? c : 0));
    return ok ? x : f32x4{0.f, 0.f, 0.f, 0.f};
  } else {
    f32x4 x;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const bool ok = c + t < D;
      const float v = row[ok ? c + t : 0];
      x[t] = ok ? v : 0.f;
    }
    return x;
  }
}

// Stores the elements c..c+3 of y that lie inside a row of D elements.
template <int MODE>
__device__ __forceinline__ void store4m(float* row, int c, int D, const f32x4& y) {
  if constexpr (MODE == 2) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
      if (c + t < D) row[c + t] = y[t];
  } else {
    if (c < D) *reinterpret_cast<f32x4*>(row + c) = y;
  }
}

// 64 rows x D of two tensors, global -> registers -> LDS (row stride D + 4
// floats: 16-byte aligned rows, and 16-byte reads of 16 consecutive rows hit
// distinct banks). Rows at or beyond N repeat row N - 1: every product that
// involves them is masked out by a select, never by a multiply, so their
// values cannot leak (and no load sits behind a branch).
template <int D, int MODE>
struct Stage {
  static constexpr int SP = D + 4;
  static constexpr int C4 = D / 4;                  // float4 per row
  static constexpr int NV = kCols * C4 / kThreads;  // float4 per thread per tensor
  static_assert(NV >= 1 && kCols * C4 % kThreads == 0, "staging shape");
  f32x4 r0[NV], r1[NV];

  // rows row0 .. row0+63 of two tensors whose row t starts at t0 + t * rs
  // (and t1 + t * rs), rows clamped to n_rows - 1
  // (Dr: the real head dim, elements of a row past it read as zeros)
  __device__ __forceinline__ void load(const float* t0, const float* t1, int row0, int n_rows,
                                       size_t rs, int Dr) {
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      const int e = threadIdx.x + kThreads * u;
      const int n = min(row0 + e / C4, n_rows - 1);
      const size_t off = (size_t)n * rs;
      r0[u] = load4m<MODE>(t0 + off, 4 * (e % C4), Dr);
      r1[u] = load4m<MODE>(t1 + off, 4 * (e % C4), Dr);
    }
  }
  __device__ __forceinline__ void store(float* s0, float* s1) const {
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      const int e = threadIdx.x + kThreads * u;
      const int at = (e / C4) * SP + 4 * (e % C4);
      *reinterpret_cast<f32x4*>(s0 + at) = r0[u];
      *reinterpret_cast<f32x4*>(s1 + at) = r1[u];
    }
  }
};

// Workgroup w takes (b, h) = w % (B*H) and row block rank w / (B*H): all
// (b, h) of one rank run before the next rank, ranks in order of decreasing
// work, so the hardware's round-robin of workgroups over the 8 XCDs gives
// every XCD the same causal load, and the blocks of one (b, h) share the L2
// of one XCD (w % 8 = (b*H + h) % 8 when B*H is a multiple of 8).

// dQ and the row deltas; rank 0 = the last query block (the most keys).
template <int D, int MODE>
__global__ __launch_bounds__(kThreads, D <= 64 ? 3 : 1) void k_fbwd_dq(FbwdArgs a) {
  constexpr int G = D / 8;             // 16-byte pairs of a row fragment
  constexpr int DT = (D + 31) / 32;    // 32-row tiles of dQ^T
  constexpr int SP = Stage<D, MODE>::SP;
  const int RS = MODE == 0 ? D : a.D;  // the real head dim: row stride, last valid column + 1
  // K and V tiles in one LDS object (one base register plus immediates)
  struct alignas(16) KV {
    float k[kCols * SP];
    float v[kCols * SP];
  };
  __shared__ KV skv;
  float* const sK = skv.k;
  float* const sV = skv.v;

  const int H = a.H, N = a.N;
  const int bh = (int)(blockIdx.x % (unsigned)a.BH), rank = (int)(blockIdx.x / (unsigned)a.BH);
  const int b = bh / H, h = bh % H;
  const int blk = a.n_blocks - 1 - rank;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 31, hf = lane >> 5;
  const int qrow = blk * kRows + wave * 32 + c;
  const bool qok = qrow < N;
  const int qr = qok ? qrow : N - 1;
  const size_t qoff = row_off(b, qr, N, H, h, RS);

  // this lane's query: Q and dO fragments (d = 8g + 4hf + t), and Dl. A lane
  // past N works on row N - 1 and masks all of its keys (qlim = -1).
  f32x4 qf[G], df[G];
  float dl = 0.f;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int d0 = 8 * g + 4 * hf;
    qf[g] = load4m<MODE>(a.q + qoff, d0, RS);
    df[g] = load4m<MODE>(a.dout + qoff, d0, RS);
    const f32x4 od = load4m<MODE>(a.o + qoff, d0, RS);
    dl += df[g].x * od.x + df[g].y * od.y + df[g].z * od.z + df[g].w * od.w;
  }
  dl = xor32_sum(dl);
  const size_t srow = (size_t)(b * N + qr) * H + h;
  if (qok && hf == 0) a.delta[srow] = dl;
  const float m2 = a.M[srow] * LOG2E;
  const float il = 1.f / a.L[srow];
  const int qlim = qok ? qrow : -1;  // keys <= qlim are unmasked

  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16{};

  const int q_last = min(blk * kRows + kRows, N) - 1;            // the workgroup's last query
  // the wave's last query (-1: the wave has none)
  const int wq_last = blk * kRows + wave * 32 < N ? min(blk * kRows + wave * 32 + 31, N - 1) : -1;
  const int steps = q_last / kCols + 1;
  const size_t rs = (size_t)H * RS;
  const float* kh = a.k + row_off(b, 0, N, H, h, RS);
  const float* vh = a.v + row_off(b, 0, N, H, h, RS);
  Stage<D, MODE> st;
  constexpr bool PF = D > 64;  // the next rows a step ahead, in registers
  if (PF) st.load(kh, vh, 0, N, rs, RS);
  for (int j = 0; j < steps; ++j) {
    if (!PF) st.load(kh, vh, j * kCols, N, rs, RS);
    __syncthreads();
    st.store(sK, sV);
    __syncthreads();
    if (PF && j + 1 < steps) st.load(kh, vh, (j + 1) * kCols, N, rs, RS);
#pragma unroll
    for (int sub = 0; sub < kCols / 32; ++sub) {
      const int key0 = j * kCols + sub * 32;
      if (key0 > wq_last) break;  // wave-uniform: every later key is masked for this wave
      f32x16 s = f32x16{}, dp = f32x16{};
      const float* kr = sK + (sub * 32 + c) * SP + 4 * hf;
      const float* vr = sV + (sub * 32 + c) * SP + 4 * hf;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const f32x4 ka = *reinterpret_cast<const f32x4*>(kr + 8 * g);
        const f32x4 va = *reinterpret_cast<const f32x4*>(vr + 8 * g);
        s = mfma(ka.x, qf[g].x, s);
        dp = mfma(va.x, df[g].x, dp);
        s = mfma(ka.y, qf[g].y, s);
        dp = mfma(va.y, df[g].y, dp);
        s = mfma(ka.z, qf[g].z, s);
        dp = mfma(va.z, df[g].z, dp);
        s = mfma(ka.w, qf[g].w, s);
        dp = mfma(va.w, df[g].w, dp);
      }
      // s[r], dp[r]: key key0 + 8(r/4) + 4hf + r%4, query qrow
      f32x16 ds;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = key0 + 8 * (r / 4) + 4 * hf + (r % 4);
        const float e = fast_exp2(s[r] * a.sl2 - m2) * il;
        const float p = key <= qlim ? e : 0.f;
        ds[r] = p * (dp[r] - dl);
      }
      // dQ^T[d][query] += sum_key K[key][d] dS^T[key][query]
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int dcol = dt * 32 + c;
        const bool dok = (MODE == 0 && D % 32 == 0) || dcol < RS;
        const float* kc = sK + (sub * 32 + 4 * hf) * SP + (dok ? dcol : RS - 1);
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float kv = kc[(8 * qq + t) * SP];
            acc[dt] = mfma(dok ? kv : 0.f, ds[4 * qq + t], acc[dt]);
          }
        }
      }
    }
  }
  // acc[dt][r]: d = dt*32 + 8(r/4) + 4hf + r%4 of this lane's query
  if (qok) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const int d0 = dt * 32 + 8 * qq + 4 * hf;
        const f32x4 y = {acc[dt][4 * qq] * a.scale, acc[dt][4 * qq + 1] * a.scale,
                         acc[dt][4 * qq + 2] * a.scale, acc[dt][4 * qq + 3] * a.scale};
        store4m<MODE>(a.dq + qoff, d0, RS, y);
      }
    }
  }
}

// dS of the five-product backward in 32 x 32 tiles: tile (query block qb, key
// block kb) of (b, h) holds 32 rows of 32 floats, row = query qb*32 + i, and
// within a row key kb*32 + 8 qq + 4 hf + t at position 16 hf + 4 qq + t: the
// order in which lane (query i, half hf) of k_fbwd_dq_ds takes the keys as
// k-steps, so that lane reads 64 contiguous bytes and a wavefront a whole
// 4 KB tile.
__device__ __forceinline__ float* ds_tile(const FbwdArgs& a, int bh, int qb, int kb) {
  const int nt = (a.N + 31) >> 5;
  return a.ds + (((size_t)bh * nt + qb) * nt + kb) * 1024;
}
__device__ __forceinline__ int ds_key_pos(int c) {  // key c of a block: 8 qq + 4 hf + t
  return 16 * ((c >> 2) & 1) + 4 * (c >> 3) + (c & 3);
}

// dK and dV; rank 0 = key block 0 (the most queries). Up to a head dim of
// 64 the workgroup's V rows wait in LDS rather than registers, so that two
// workgroups fit a CU (two wavefronts per SIMD).
template <int D>
constexpr bool fbwd_v_in_lds() { return D <= 64; }
template <int D, int MODE, bool DSO = false>  // DSO: also write dS (a.ds) for k_fbwd_dq_ds
__global__ __launch_bounds__(kThreads, fbwd_v_in_lds<D>() ? 2 : 1) void k_fbwd_dkv(FbwdArgs a) {
  constexpr int G = D / 8;
  constexpr int DT = (D + 31) / 32;
  constexpr int SP = Stage<D, MODE>::SP;
  constexpr bool VL = fbwd_v_in_lds<D>();
  const int RS = MODE == 0 ? D : a.D;  // the real head dim
  // One LDS object: the arrays sit at fixed offsets from each other, so a
  // lane's addresses into all of them are one register plus immediates (as
  // separate objects the compiler kept a register per array and spilled some)
  struct alignas(16) Smem {
    float q[kCols * SP];
    float d[kCols * SP];  // dO
    float m2[kCols], il[kCols], dl[kCols];
    float v[VL ? kRows * SP : 4];  // the block's V rows
  };
  __shared__ Smem sm;
  float* const sQ = sm.q;
  float* const sD = sm.d;
  float* const sV = sm.v;
  float* const sM2 = sm.m2;
  float* const sIL = sm.il;
  float* const sDL = sm.dl;

  const int H = a.H, N = a.N;
  const int bh = (int)(blockIdx.x % (unsigned)a.BH), rank = (int)(blockIdx.x / (unsigned)a.BH);
  const int b = bh / H, h = bh % H;
  const int blk = rank;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 31, hf = lane >> 5;
  const int wk0 = blk * kRows + wave * 32;  // the wave's first key
  const int krow = wk0 + c;  // a key past N is masked for every query (query < N <= krow)
  const size_t koff = row_off(b, min(krow, N - 1), N, H, h, RS);

  f32x4 kf[G], vf[VL ? 1 : G];
  float* vrow = sV + (VL ? (wave * 32 + c) * SP + 4 * hf : 0);  // V fragment g: vrow[8 g ..]
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int d0 = 8 * g + 4 * hf;
    kf[g] = load4m<MODE>(a.k + koff, d0, RS);
    if constexpr (VL) *reinterpret_cast<f32x4*>(vrow + 8 * g) = load4m<MODE>(a.v + koff, d0, RS);
    else vf[g] = load4m<MODE>(a.v + koff, d0, RS);
  }
  f32x16 dva[DT], dka[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    dva[dt] = f32x16{};
    dka[dt] = f32x16{};
  }
  // DSO: this lane's place in the dS tiles of its key block (query block 0;
  // the query block adds a whole row of tiles): key c, rows 4 hf + ...
  float* dsw = nullptr;
  if constexpr (DSO)
    dsw = ds_tile(a, bh, 0, wk0 >> 5) + ds_key_pos(c) + 128 * hf;

  const int j0 = (blk * kRows) / kCols;  // first step holding a query >= the block's first key
  const int steps = (N + kCols - 1) / kCols;
  Stage<D, MODE> st;
  // statistics of query j * kCols + threadIdx.x (threads < kCols), clamped
  float m2 = 0.f, il = 0.f, dl = 0.f;
#define SKV_FB_STATS(J)                                                          \
  if (threadIdx.x < kCols) {                                                     \
    const int n_ = min((J) * kCols + (int)threadIdx.x, N - 1);                   \
    const size_t sr_ = (size_t)(b * N + n_) * H + h;                             \
    m2 = a.M[sr_] * LOG2E;                                                       \
    il = 1.f / a.L[sr_];                                                         \
    dl = a.delta[sr_];                                                           \
  }
  const size_t rs = (size_t)H * RS;
  const float* qh = a.q + row_off(b, 0, N, H, h, RS);
  const float* dh = a.dout + row_off(b, 0, N, H, h, RS);
  // With V in LDS (two workgroups a CU) the next rows are loaded at the top
  // of each step, the other workgroup's products covering the wait; with one
  // workgroup a CU they are loaded a step ahead, into registers.
  if (!VL && j0 < steps) {
    st.load(qh, dh, j0 * kCols, N, rs, RS);
    SKV_FB_STATS(j0)
  }
  for (int j = j0; j < steps; ++j) {
    if (VL) {
      st.load(qh, dh, j * kCols, N, rs, RS);
      SKV_FB_STATS(j)
    }
    __syncthreads();
    st.store(sQ, sD);
    if (threadIdx.x < kCols) {
      sM2[threadIdx.x] = m2;
      sIL[threadIdx.x] = il;
      sDL[threadIdx.x] = dl;
    }
    __syncthreads();
    if (!VL && j + 1 < steps) {
      st.load(qh, dh, (j + 1) * kCols, N, rs, RS);
      SKV_FB_STATS(j + 1)
    }
#pragma unroll
    for (int sub = 0; sub < kCols / 32; ++sub) {
      const int q0 = j * kCols + sub * 32;
      // wave-uniform: every query precedes the wave's keys, or the wave has no key
      if (q0 + 31 < wk0 || wk0 >= N) continue;
      f32x16 s = f32x16{}, dp = f32x16{};
      const float* qr = sQ + (sub * 32 + c) * SP + 4 * hf;
      const float* dr = sD + (sub * 32 + c) * SP + 4 * hf;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const f32x4 qa = *reinterpret_cast<const f32x4*>(qr + 8 * g);
        const f32x4 da = *reinterpret_cast<const f32x4*>(dr + 8 * g);
        f32x4 vg;
        if constexpr (VL) vg = *reinterpret_cast<const f32x4*>(vrow + 8 * g);
        else vg = vf[g];
        s = mfma(qa.x, kf[g].x, s);
        dp = mfma(da.x, vg.x, dp);
        s = mfma(qa.y, kf[g].y, s);
        dp = mfma(da.y, vg.y, dp);
        s = mfma(qa.z, kf[g].z, s);
        dp = mfma(da.z, vg.z, dp);
        s = mfma(qa.w, kf[g].w, s);
        dp = mfma(da.w, vg.w, dp);
      }
      // s[r], dp[r]: query q0 + 8(r/4) + 4hf + r%4, key krow
      f32x16 p, ds;
      // wave-uniform: every key of the wave precedes every query of the
      // piece and every query exists, so no slot is masked or skipped
      const bool interior = q0 >= wk0 + 31 && q0 + 32 <= N;
      if (interior) {
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const int ql = sub * 32 + 8 * qq + 4 * hf;
          const f32x4 m4 = *reinterpret_cast<const f32x4*>(sM2 + ql);
          const f32x4 i4 = *reinterpret_cast<const f32x4*>(sIL + ql);
          const f32x4 d4 = *reinterpret_cast<const f32x4*>(sDL + ql);
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int r = 4 * qq + t;
            const float e = fast_exp2(s[r] * a.sl2 - m4[t]) * i4[t];
            p[r] = e;
            ds[r] = e * (dp[r] - d4[t]);
          }
        }
      } else {
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const int ql = sub * 32 + 8 * qq + 4 * hf;
          const f32x4 m4 = *reinterpret_cast<const f32x4*>(sM2 + ql);
          const f32x4 i4 = *reinterpret_cast<const f32x4*>(sIL + ql);
          const f32x4 d4 = *reinterpret_cast<const f32x4*>(sDL + ql);
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int r = 4 * qq + t, query = j * kCols + ql + t;
            const float e = fast_exp2(s[r] * a.sl2 - m4[t]) * i4[t];
            const float pr = (krow <= query && query < N) ? e : 0.f;
            p[r] = pr;
            ds[r] = pr * (dp[r] - d4[t]);
          }
        }
      }
      if constexpr (DSO) {
        // dS of the piece (query block q0 / 32, key block wk0 / 32) for
        // k_fbwd_dq_ds, in the order its lanes read: for each slot the 32
        // lanes of a half write one query's 128-byte tile row
        if (krow < N) {
          float* tp = dsw + (size_t)(q0 >> 5) * ((N + 31) >> 5) * 1024;
          if (q0 + 32 <= N) {  // wave-uniform: every row of the tile exists
#pragma unroll
            for (int r = 0; r < 16; ++r)
              __builtin_nontemporal_store(ds[r], tp + (8 * (r / 4) + (r % 4)) * 32);
          } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int qi = 8 * (r / 4) + 4 * hf + (r % 4);  // query q0 + qi
              if (q0 + qi < N)  // row qi of the tile; streamed past the caches (read once, later)
                __builtin_nontemporal_store(ds[r], tp + (8 * (r / 4) + (r % 4)) * 32);
            }
          }
        }
      }
      // dV[key][d] += sum_query P^T[key][query] dO[query][d]; dK likewise with dS and Q
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int dcol = dt * 32 + c;
        const bool dok = (MODE == 0 && D % 32 == 0) || dcol < RS;
        const int at = (sub * 32 + 4 * hf) * SP + (dok ? dcol : RS - 1);
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float xo = sD[at + (8 * qq + t) * SP];
            const float xq = sQ[at + (8 * qq + t) * SP];
            dva[dt] = mfma(p[4 * qq + t], dok ? xo : 0.f, dva[dt]);
            dka[dt] = mfma(ds[4 * qq + t], dok ? xq : 0.f, dka[dt]);
          }
        }
      }
    }
  }
#undef SKV_FB_STATS
  // dva[dt][r], dka[dt][r]: key wk0 + 8(r/4) + 4hf + r%4, d = dt*32 + c
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    const int d = dt * 32 + c;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = wk0 + 8 * (r / 4) + 4 * hf + (r % 4);
      if (key < N && ((MODE == 0 && D % 32 == 0) || d < RS)) {
        const size_t off = row_off(b, key, N, H, h, RS) + d;
        a.dk[off] = dka[dt][r] * a.scale;
        a.dv[off] = dva[dt][r];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Forward: causal attention with the forward's row statistics, fp32.
// ---------------------------------------------------------------------------

struct FfwdArgs {
  const float* q;  // [B, C, Hq, D]
  const float* k;  // [B, T_cap, Hkv, D]
  const float* v;
  const int32_t* start;  // per-sequence position of query 0 (NULL: 0)
  const int32_t* n_new;  // per-sequence valid queries (NULL: C)
  float* out;            // [B, C, Hq, D]; rows i >= n_new[b] get zeros
  float* L;              // [B, C, Hq] softmax sums (may be NULL)
  float* M;              // [B, C, Hq] row maxima of the scaled scores (may be NULL)
  int C, Hq, Hkv, T_cap, BH, n_blocks;
  int D;  // head dim (the padded size is the kernel's template D)
  float sl2;  // scale * log2(e)
};

// One workgroup per (128 queries, b, query head); rank-major order as in the
// backward. Each wave owns 32 queries (lane c, both halves): per 32-key piece
// S^T = K Q^T, an online softmax over the piece, then O^T += V^T P^T. The
// running max moves only when a piece's max exceeds it by more than 8 (log2
// units), so O and l are rescaled on few pieces; the true maximum is kept
// beside it for M and the final L.
template <int D, int MODE>
__global__ __launch_bounds__(kThreads, D <= 64 ? 3 : 1) void k_flash_fwd(FfwdArgs a) {
  constexpr int G8 = D / 8;
  constexpr int DT = (D + 31) / 32;
  constexpr int SP = Stage<D, MODE>::SP;
  const int RS = MODE == 0 ? D : a.D;  // the real head dim
  // K and V tiles in one LDS object (one base register plus immediates)
  struct alignas(16) KV {
    float k[kCols * SP];
    float v[kCols * SP];
  };
  __shared__ KV skv;
  float* const sK = skv.k;
  float* const sV = skv.v;

  const int Hq = a.Hq, C = a.C;
  const int bh = (int)(blockIdx.x % (unsigned)a.BH), rank = (int)(blockIdx.x / (unsigned)a.BH);
  const int b = bh / Hq, h = bh % Hq, hk = h / (Hq / a.Hkv);
  const int blk = a.n_blocks - 1 - rank;
  const int P = a.start ? min(max(a.start[b], 0), a.T_cap) : 0;
  const int n = max(0, min(a.n_new ? min(a.n_new[b], C) : C, a.T_cap - P));  // valid queries
  const int kv_end = P + n;  // keys [0, kv_end) exist
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 31, hf = lane >> 5;
  const int qi = blk * kRows + wave * 32 + c;  // this lane's query (row of the chunk)
  const bool qok = qi < n;
  const int qlim = qok ? P + qi : -1;          // keys <= qlim are unmasked
  const size_t qoff = (((size_t)b * C + min(qi, max(n, 1) - 1)) * Hq + h) * RS;

  f32x4 qf[G8];
#pragma unroll
  for (int g = 0; g < G8; ++g) qf[g] = load4m<MODE>(a.q + qoff, 8 * g + 4 * hf, RS);
  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16{};
  float m_run = -INFINITY, m_true = -INFINITY, l = 0.f;

  // keys this workgroup and this wave need
  const int blk_q = min(blk * kRows + kRows, n);  // valid queries of the block end here
  const int steps = blk * kRows < n ? (P + blk_q + kCols - 1) / kCols : 0;
  const int wq0 = blk * kRows + wave * 32;  // the wave's first query
  const bool wfull = wq0 + 31 < n;           // all 32 of its queries valid
  const int wq_last = wq0 < n ? P + min(wq0 + 31, n - 1) : -1;
  const size_t rs = (size_t)a.Hkv * RS;
  const float* kh = a.k + ((size_t)b * a.T_cap * a.Hkv + hk) * RS;
  const float* vh = a.v + ((size_t)b * a.T_cap * a.Hkv + hk) * RS;
  Stage<D, MODE> st;
  if (steps > 0) st.load(kh, vh, 0, kv_end, rs, RS);
  for (int j = 0; j < steps; ++j) {
    __syncthreads();
    st.store(sK, sV);
    __syncthreads();
    if (j + 1 < steps) st.load(kh, vh, (j + 1) * kCols, kv_end, rs, RS);
#pragma unroll
    for (int sub = 0; sub < kCols / 32; ++sub) {
      const int key0 = j * kCols + sub * 32;
      if (key0 > wq_last) break;  // wave-uniform: every later key is masked for this wave
      f32x16 s = f32x16{};
      const float* kr = sK + (sub * 32 + c) * SP + 4 * hf;
#pragma unroll
      for (int g = 0; g < G8; ++g) {
        const f32x4 ka = *reinterpret_cast<const f32x4*>(kr + 8 * g);
        s = mfma(ka.x, qf[g].x, s);
        s = mfma(ka.y, qf[g].y, s);
        s = mfma(ka.z, qf[g].z, s);
        s = mfma(ka.w, qf[g].w, s);
      }
      // s[r]: key key0 + 8(r/4) + 4hf + r%4 of this lane's query, in log2 units.
      // A piece wholly at or below the diagonal of a wave whose 32 queries
      // are all valid masks nothing (wave-uniform test).
      float tmax = -INFINITY;
      if (wfull && key0 + 31 <= P + wq0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          s[r] *= a.sl2;
          tmax = fmaxf(tmax, s[r]);
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = key0 + 8 * (r / 4) + 4 * hf + (r % 4);
          s[r] = key <= qlim ? s[r] * a.sl2 : -INFINITY;
          tmax = fmaxf(tmax, s[r]);
        }
      }
      tmax = xor32_max(tmax);  // both halves hold the same query
      m_true = fmaxf(m_true, tmax);
      const bool upd = tmax > m_run + 8.f;  // also true on the first piece with a key
      if (__ballot(upd) != 0ull) {          // wave-uniform branch
        const float alpha = upd ? fast_exp2(m_run - tmax) : 1.f;  // m_run = -inf: 0
        if (upd) m_run = tmax;
        l *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
      }
      const float m_use = m_run == -INFINITY ? 0.f : m_run;  // nothing unmasked yet
      f32x16 p;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        p[r] = fast_exp2(s[r] - m_use);
        l += p[r];
      }
      // O^T[d][query] += sum_key V[key][d] P^T[key][query]
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int dcol = dt * 32 + c;
        const bool dok = (MODE == 0 && D % 32 == 0) || dcol < RS;
        const float* vc = sV + (sub * 32 + 4 * hf) * SP + (dok ? dcol : RS - 1);
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float vv = vc[(8 * qq + t) * SP];
            acc[dt] = mfma(dok ? vv : 0.f, p[4 * qq + t], acc[dt]);
          }
        }
      }
    }
  }
  const float lt = xor32_sum(l);
  if (qi >= C) return;
  const size_t orow = ((size_t)b * C + qi) * Hq + h;
  const float inv = qok ? 1.f / lt : 0.f;  // a valid row saw its own key: lt >= 1
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const int d0 = dt * 32 + 8 * qq + 4 * hf;
      const f32x4 y = {acc[dt][4 * qq] * inv, acc[dt][4 * qq + 1] * inv,
                       acc[dt][4 * qq + 2] * inv, acc[dt][4 * qq + 3] * inv};
      store4m<MODE>(a.out + orow * RS, d0, RS, y);
    }
  }
  if (hf == 0 && qok) {
    if (a.L) a.L[orow] = lt * fast_exp2(m_run - m_true);  // relative to the true maximum
    if (a.M) a.M[orow] = m_true * (1.f / LOG2E);          // natural units, as the scores
  }
}

// ---------------------------------------------------------------------------
// The five-product backward (head dims up to 64, a workspace that holds dS):
// k_fbwd_delta writes the row deltas, k_fbwd_dkv also writes dS = P * (dP -
// Dl) of every (query, key <= query) piece it forms, and k_fbwd_dq_ds forms
// dQ = scale * dS K from it, so dQ no longer recomputes S and dP (7 products
// -> 5, at the cost of writing and reading dS once: B * H * N^2 / 2 floats).
// ---------------------------------------------------------------------------

// Dl = rowsum(dO * O): 16 lanes per (b, n, h) row, lane i = 2 g + hf holding
// elements 8 g + 4 hf .. + 3 (coalesced: a row's lanes read its 256 bytes);
// the sums are taken as k_fbwd_dq takes them (each half's fragments in order
// of g, then the two halves), so Dl has the same bits.
template <int D, int MODE>
__global__ __launch_bounds__(256) void k_fbwd_delta(FbwdArgs a, long rows) {
  const long row = ((long)blockIdx.x * 256 + threadIdx.x) >> 4;
  const int i = threadIdx.x & 15;  // lane in the row
  const long rr = row < rows ? row : rows - 1;
  const int RS = MODE == 0 ? D : a.D;
  float t = 0.f;
  if (i < D / 4) {  // D / 8 groups of two halves: D / 4 lanes
    const int d0 = 8 * (i >> 1) + 4 * (i & 1);
    const f32x4 x = load4m<MODE>(a.dout + (size_t)rr * RS, d0, RS);
    const f32x4 y = load4m<MODE>(a.o + (size_t)rr * RS, d0, RS);
    t = x.x * y.x + x.y * y.y + x.z * y.z + x.w * y.w;
  }
  float half[2] = {0.f, 0.f};
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int g = 0; g < D / 8; ++g) half[hf] += __shfl(t, (threadIdx.x & 48) + 2 * g + hf, 64);
  if (i == 0 && row < rows) a.delta[row] = half[0] + half[1];
}

// dQ from the stored dS: one workgroup per (128 queries, b, h), rank 0 = the
// last query block; each wave owns 32 queries. Per 32-key piece the lane of
// query c loads its dS row's keys 8 qq + 4 hf .. + 3 (the k-steps of the
// product, as k_fbwd_dq orders them) one piece ahead, and K goes through LDS
// 64 rows at a time. dS of a key past the query (or past N) is masked by a
// select: k_fbwd_dkv wrote zeros there only for the pieces it formed.
template <int D, int MODE>
__global__ __launch_bounds__(kThreads) void k_fbwd_dq_ds(FbwdArgs a) {
  constexpr int DT = (D + 31) / 32;
  constexpr int SP = D + 4;
  constexpr int C4 = D / 4;
  constexpr int NV = kCols * C4 / kThreads;  // float4 of K per thread per step
  const int RS = MODE == 0 ? D : a.D;
  __shared__ __attribute__((aligned(16))) float sK[kCols * SP];

  const int H = a.H, N = a.N;
  const int bh = (int)(blockIdx.x % (unsigned)a.BH), rank = (int)(blockIdx.x / (unsigned)a.BH);
  const int b = bh / H, h = bh % H;
  const int blk = a.n_blocks - 1 - rank;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 31, hf = lane >> 5;
  const int qrow = blk * kRows + wave * 32 + c;
  const bool qok = qrow < N;
  const int qr = qok ? qrow : N - 1;
  const int qlim = qok ? qrow : -1;  // keys <= qlim are unmasked
  const int qb = blk * 4 + wave;  // the wave's query block

  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16{};
  const int q_last = min(blk * kRows + kRows, N) - 1;
  const int wq_last = blk * kRows + wave * 32 < N ? min(blk * kRows + wave * 32 + 31, N - 1) : -1;
  const int steps = q_last / kCols + 1;
  const size_t rs = (size_t)H * RS;
  const float* kh = a.k + row_off(b, 0, N, H, h, RS);

  // dS of the piece at key0 for this lane: keys key0 + 8 qq + 4 hf + t, 64
  // contiguous bytes of the tile, loaded a piece ahead; masked only where it
  // is used (a select there, not here, so the load is not waited for at once)
  auto load_ds = [&](int key0, f32x4 (&x)[4]) {
    const float* tp = ds_tile(a, bh, qb, key0 >> 5) + c * 32 + 16 * hf;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) x[qq] = *reinterpret_cast<const f32x4*>(tp + 4 * qq);
  };
  f32x4 cur[4], nxt[4] = {};
  if (wq_last >= 0) load_ds(0, cur);
  f32x4 kr[NV];  // the next step's K rows, loaded a step ahead
  auto load_k = [&](int j) {
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      const int e = threadIdx.x + kThreads * u;
      const int n = min(j * kCols + e / C4, N - 1);
      kr[u] = load4m<MODE>(kh + (size_t)n * rs, 4 * (e % C4), RS);
    }
  };
  load_k(0);
  for (int j = 0; j < steps; ++j) {
    __syncthreads();
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      const int e = threadIdx.x + kThreads * u;
      *reinterpret_cast<f32x4*>(sK + (e / C4) * SP + 4 * (e % C4)) = kr[u];
    }
    __syncthreads();
    if (j + 1 < steps) load_k(j + 1);
#pragma unroll
    for (int sub = 0; sub < kCols / 32; ++sub) {
      const int key0 = j * kCols + sub * 32;
      if (key0 > wq_last) break;  // wave-uniform: every later key is masked for this wave
      if (key0 + 32 <= wq_last) load_ds(key0 + 32, nxt);
      // keys past the query (or past N: entries never written) weigh 0, by a select
#pragma unroll
      for (int qq = 0; qq < 4; ++qq)
#pragma unroll
        for (int t = 0; t < 4; ++t)
          cur[qq][t] = key0 + 8 * qq + 4 * hf + t <= qlim ? cur[qq][t] : 0.f;
      // dQ^T[d][query] += sum_key K[key][d] dS^T[key][query]
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int dcol = dt * 32 + c;
        const bool dok = (MODE == 0 && D % 32 == 0) || dcol < RS;
        const float* kc = sK + (sub * 32 + 4 * hf) * SP + (dok ? dcol : RS - 1);
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float kv = kc[(8 * qq + t) * SP];
            acc[dt] = mfma(dok ? kv : 0.f, cur[qq][t], acc[dt]);
          }
        }
      }
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) cur[qq] = nxt[qq];
    }
  }
  if (qok) {
    const size_t qoff = row_off(b, qr, N, H, h, RS);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const int d0 = dt * 32 + 8 * qq + 4 * hf;
        const f32x4 y = {acc[dt][4 * qq] * a.scale, acc[dt][4 * qq + 1] * a.scale,
                         acc[dt][4 * qq + 2] * a.scale, acc[dt][4 * qq + 3] * a.scale};
        store4m<MODE>(a.dq + qoff, d0, RS, y);
      }
    }
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Padded head dim and load mode of a head dim: a multiple of 16 up to 128,
// then 192 or 256 (the forward only: one wavefront per SIMD holds a 256-wide
// query row set and its accumulators without spilling; the backward's
// kernels hold two row operands and an accumulator and stop at 128).
struct FlashShape {
  int DP, mode;
};
FlashShape flash_shape(int D) {
  const int DP = D <= 128 ? (D + 15) / 16 * 16 : D <= 192 ? 192 : 256;
  return {DP, D == DP ? 0 : (D % 4 == 0 ? 1 : 2)};
}

// Expands X(DP, MODE) for every kernel shape.
#define SKV_FLASH_SHAPES(X)                                                           \
  X(16, 0) X(16, 1) X(16, 2) X(32, 0) X(32, 1) X(32, 2) X(48, 0) X(48, 1) X(48, 2)    \
  X(64, 0) X(64, 1) X(64, 2) X(80, 0) X(80, 1) X(80, 2) X(96, 0) X(96, 1) X(96, 2)    \
  X(112, 0) X(112, 1) X(112, 2) X(128, 0) X(128, 1) X(128, 2)
// The shapes past 128 (the forward's here; the backward's in the wide
// translation unit).
#define SKV_FLASH_WIDE_SHAPES(X) X(192, 0) X(192, 1) X(192, 2) X(256, 0) X(256, 1) X(256, 2)

FbwdArgs fbwd_args(float* dq, float* dk, float* dv, const float* q, const float* k,
                   const float* v, const float* o, const float* L, const float* M,
                   const float* dout, float* delta, int B, int N, int H, int D, float scale) {
  FbwdArgs a;
  a.q = q; a.k = k; a.v = v; a.o = o; a.dout = dout; a.L = L; a.M = M;
  a.dq = dq; a.dk = dk; a.dv = dv;
  a.delta = delta;
  a.ds = nullptr;
  a.N = N; a.H = H; a.D = D;
  a.n_blocks = (N + kRows - 1) / kRows;
  a.scale = scale;
  a.sl2 = scale * LOG2E;
  a.BH = B * H;
  return a;
}

// The two backward kernels of shape fs (one of SHAPES) for a.
#define SKV_FB(DD, MM)                                                             \
  if (fs.DP == DD && fs.mode == MM) {                                              \
    hipLaunchKernelGGL((k_fbwd_dq<DD, MM>), grid, dim3(kThreads), 0, s, a);        \
    int rc = check_launch("skv_flash_bwd");                                        \
    if (rc) return rc;                                                             \
    hipLaunchKernelGGL((k_fbwd_dkv<DD, MM>), grid, dim3(kThreads), 0, s, a);       \
    return check_launch("skv_flash_bwd");                                          \
  }

}  // namespace

#if SKV_FLASH_WIDE_BWD
// The backward past a head dim of 128 (padded to 192 or 256). This
// translation unit is the same source built without -amdgpu-mfma-vgpr-form:
// each wavefront holds two 32-row operands and an accumulator of the head
// dim, more than the VGPRs alone (the MFMA accumulators then live in AGPRs;
// the rest spills to scratch, so these shapes run correctly but far below
// the narrow ones' rate).
int fbwd_wide(float* dq, float* dk, float* dv, const float* q, const float* k, const float* v,
              const float* o, const float* L, const float* M, const float* dout, float* delta,
              int B, int N, int H, int D, float scale, int DP, int mode, hipStream_t s) {
  const FbwdArgs a = fbwd_args(dq, dk, dv, q, k, v, o, L, M, dout, delta, B, N, H, D, scale);
  const FlashShape fs{DP, mode};
  const dim3 grid((unsigned)(a.n_blocks * a.BH));
  SKV_FLASH_WIDE_SHAPES(SKV_FB)
  return set_error(SKV_E_UNSUPPORTED, "skv_flash_bwd: no kernel for head_dim %d", D);
}
#else
namespace {
int fbwd_launch(const FbwdArgs& a, const FlashShape& fs, hipStream_t s) {
  const dim3 grid((unsigned)(a.n_blocks * a.BH));
  SKV_FLASH_SHAPES(SKV_FB)
  return set_error(SKV_E_UNSUPPORTED, "skv_flash_bwd: no kernel for head_dim %d", a.D);
}

// The five-product backward (a.ds set): row deltas, dK/dV with dS written,
// then dQ from dS.
#define SKV_FB_DS(DD, MM)                                                            \
  if (fs.DP == DD && fs.mode == MM) {                                                \
    hipLaunchKernelGGL((k_fbwd_delta<DD, MM>), dim3((unsigned)((rows + 15) / 16)),    \
                       dim3(256), 0, s, a, rows);                                    \
    int rc = check_launch("skv_flash_bwd");                                          \
    if (rc) return rc;                                                               \
    hipLaunchKernelGGL((k_fbwd_dkv<DD, MM, true>), grid, dim3(kThreads), 0, s, a);   \
    rc = check_launch("skv_flash_bwd");                                              \
    if (rc) return rc;                                                               \
    hipLaunchKernelGGL((k_fbwd_dq_ds<DD, MM>), grid, dim3(kThreads), 0, s, a);       \
    return check_launch("skv_flash_bwd");                                            \
  }
int fbwd_launch_ds(const FbwdArgs& a, const FlashShape& fs, long rows, hipStream_t s) {
  const dim3 grid((unsigned)(a.n_blocks * a.BH));
  SKV_FB_DS(16, 0) SKV_FB_DS(16, 1) SKV_FB_DS(16, 2) SKV_FB_DS(32, 0) SKV_FB_DS(32, 1)
  SKV_FB_DS(32, 2) SKV_FB_DS(48, 0) SKV_FB_DS(48, 1) SKV_FB_DS(48, 2) SKV_FB_DS(64, 0)
  SKV_FB_DS(64, 1) SKV_FB_DS(64, 2)
  return set_error(SKV_E_UNSUPPORTED, "skv_flash_bwd: no kernel for head_dim %d", a.D);
}
#undef SKV_FB_DS

// Workspace of the five-product backward: the row deltas (256-byte
// aligned block), then dS; 0 where that path does not apply.
size_t fbwd_ds_bytes(int B, int N, int H, int D) {
  if (B <= 0 || N <= 0 || H <= 0 || D <= 0 || D > 64) return 0;
  const size_t dl = ((size_t)B * N * H * sizeof(float) + 255) / 256 * 256;
  const size_t n32 = ((size_t)N + 31) / 32 * 32;  // N in whole 32 x 32 tiles
  return dl + (size_t)B * H * n32 * n32 * sizeof(float);
}
}  // namespace
#endif
#undef SKV_FB
}  // namespace skv

#if !SKV_FLASH_WIDE_BWD

using namespace skv;

extern "C" size_t skv_flash_bwd_workspace_bytes(int B, int N, int H) {
  if (B <= 0 || N <= 0 || H <= 0) return 0;
  return (size_t)B * N * H * sizeof(float);
}

extern "C" size_t skv_flash_bwd_fast_workspace_bytes(int B, int N, int H, int D) {
  const size_t fast = fbwd_ds_bytes(B, N, H, D);
  return fast ? fast : skv_flash_bwd_workspace_bytes(B, N, H);
}

extern "C" int skv_flash_bwd(float* dq, float* dk, float* dv, const float* q, const float* k,
                             const float* v, const float* o, const float* L, const float* M,
                             const float* dout, int B, int N, int H, int D, float scale, void* ws,
                             size_t ws_bytes, skv_stream_t stream) {
  const char* fn = "skv_flash_bwd";
  SKV_REQUIRE(dq && dk && dv && q && k && v && o && L && M && dout, SKV_E_INVALID,
              "%s: null pointer argument", fn);
  SKV_REQUIRE(B > 0 && N > 0 && H > 0 && D > 0, SKV_E_INVALID,
              "%s: dims must be > 0 (B=%d N=%d H=%d D=%d)", fn, B, N, H, D);
  SKV_REQUIRE(D <= 256, SKV_E_UNSUPPORTED, "%s: head_dim %d (supported: 1 to 256)", fn, D);
  SKV_REQUIRE(scale > 0.f, SKV_E_INVALID, "%s: scale must be > 0", fn);
  SKV_REQUIRE(aligned16(dq) && aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o) &&
                  aligned16(dout),
              SKV_E_INVALID, "%s: q, k, v, o, dout and dq must be 16-byte aligned", fn);
  SKV_REQUIRE((long)B * N * H * D < (1L << 40), SKV_E_UNSUPPORTED, "%s: tensors too large", fn);
  const size_t need = skv_flash_bwd_workspace_bytes(B, N, H);
  SKV_REQUIRE(ws && ws_bytes >= need && aligned16(ws), SKV_E_WORKSPACE,
              "%s: workspace %zu bytes < %zu required (16-byte aligned)", fn, ws_bytes, need);
  const FbwdArgs a = fbwd_args(dq, dk, dv, q, k, v, o, L, M, dout, static_cast<float*>(ws), B,
                               N, H, D, scale);
  hipStream_t s = (hipStream_t)stream;
  SKV_REQUIRE((long)a.n_blocks * a.BH < (1L << 31), SKV_E_UNSUPPORTED, "%s: grid too large", fn);
  const FlashShape fs = flash_shape(D);
  if (fs.DP > 128)  // kernels of the wide translation unit
    return fbwd_wide(dq, dk, dv, q, k, v, o, L, M, dout, a.delta, B, N, H, D, scale, fs.DP,
                     fs.mode, s);
  const size_t fast = fbwd_ds_bytes(B, N, H, D);
  if (fast && ws_bytes >= fast) {  // room for dS: the five-product path
    FbwdArgs ad = a;
    ad.ds = reinterpret_cast<float*>(static_cast<char*>(ws) +
                                     ((size_t)B * N * H * sizeof(float) + 255) / 256 * 256);
    return fbwd_launch_ds(ad, fs, (long)B * N * H, s);
  }
  return fbwd_launch(a, fs, s);
}

namespace skv {

// Causal fp32 attention of C queries per sequence over the keys [0, start[b]
// + i] of a [B, T_cap, Hkv, D] key/value layout (shared by skv_flash_fwd and
// skv_prefill_attn on fp32 caches). Pointers are checked by the callers.
int attn_fwd_f32(float* out, float* L, float* M, const float* q, const float* k, const float* v,
                 const int32_t* start, const int32_t* n_new, int B, int C, int Hq, int Hkv, int D,
                 int T_cap, float scale, hipStream_t s, const char* fn) {
  SKV_REQUIRE(D >= 1 && D <= 256, SKV_E_UNSUPPORTED, "%s: head_dim %d (supported: 1 to 256)",
              fn, D);
  SKV_REQUIRE(aligned16(out) && aligned16(q) && aligned16(k) && aligned16(v), SKV_E_INVALID,
              "%s: q, k, v and out must be 16-byte aligned", fn);
  FfwdArgs a;
  a.q = q; a.k = k; a.v = v; a.start = start; a.n_new = n_new;
  a.out = out; a.L = L; a.M = M;
  a.C = C; a.Hq = Hq; a.Hkv = Hkv; a.T_cap = T_cap; a.D = D;
  a.BH = B * Hq;
  a.n_blocks = (C + kRows - 1) / kRows;
  a.sl2 = scale * LOG2E;
  SKV_REQUIRE((long)a.n_blocks * a.BH < (1L << 31), SKV_E_UNSUPPORTED, "%s: grid too large", fn);
  const dim3 grid((unsigned)(a.n_blocks * a.BH));
  const FlashShape fs = flash_shape(D);
#define SKV_FF(DD, MM) \
  if (fs.DP == DD && fs.mode == MM) hipLaunchKernelGGL((k_flash_fwd<DD, MM>), grid, dim3(kThreads), 0, s, a);
  SKV_FLASH_SHAPES(SKV_FF)
  SKV_FLASH_WIDE_SHAPES(SKV_FF)
#undef SKV_FF
  return check_launch(fn);
}

}  // namespace skv

extern "C" int skv_flash_fwd(float* out, float* L, float* M, const float* q, const float* k,
                             const float* v, int B, int N, int H, int D, float scale,
                             skv_stream_t stream) {
  const char* fn = "skv_flash_fwd";
  SKV_REQUIRE(out && q && k && v, SKV_E_INVALID, "%s: null pointer argument", fn);
  SKV_REQUIRE(B > 0 && N > 0 && H > 0 && D > 0, SKV_E_INVALID,
              "%s: dims must be > 0 (B=%d N=%d H=%d D=%d)", fn, B, N, H, D);
  SKV_REQUIRE(scale > 0.f, SKV_E_INVALID, "%s: scale must be > 0", fn);
  SKV_REQUIRE((long)B * N * H * D < (1L << 40), SKV_E_UNSUPPORTED, "%s: tensors too large", fn);
  return attn_fwd_f32(out, L, M, q, k, v, nullptr, nullptr, B, N, H, H, D, N, scale,
                      (hipStream_t)stream, fn);
}
#endif  // !SKV_FLASH_WIDE_BWD
