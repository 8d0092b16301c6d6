// Pass 1 of cached decode attention with grouped queries on the matrix
// cores: bf16 caches, head dim 64 or 128, G = H_q / H_kv in {2, 4, 8}.
//
// Same work split, partial format and merge pass as the VALU kernels
// (decode_kernels.h): workgroup w owns tokens [w*chunk, (w+1)*chunk) of the
// flat token stream, cut into pieces at sequence boundaries, and writes one
// partial (m, l, o[D]) per (piece, query head) at slot w + b. What differs is
// how a wavefront consumes a piece. With G query heads per kv head the VALU
// kernels spend ~36 wavefront instructions per (token, kv head) on the q.k
// dots, the p.V updates and their cross-lane sums; here both products run
// on v_mfma_f32_16x16x32_bf16 and the VALU is left with the softmax itself
// (~3 instructions per token and kv head), so the pass is bound by HBM.
//
// One wavefront serves one kv head and G query heads, in steps of 32 tokens
// (two 16-token tiles):
//  * S = K q^T: operand A is the K tile straight from HBM (lane l holds row
//    l%16, 8 consecutive elements per k-block), operand B is the query:
//    column c < G holds head c, column G + c holds head c again, and the k
//    dimension is [D elements of q_hi ; D elements of q_lo], q_hi =
//    bf16(q * scale * log2 e), q_lo = bf16(that - q_hi), against [K | K].
//    The split makes q.k exact to ~2^-17 relative (K is bf16 already), and
//    the duplicated columns give both column c and G + c the full score of
//    head c, bit for bit.
//  * Online softmax per column, lanes of column c holding 8 of the step's
//    32 scores. The running max is kept lazily: the accumulator is rescaled
//    only when a step's max exceeds it by more than 8 (log2 units), so p =
//    exp2(s - m) <= 256; (m, l, o) stay consistent, the merge is exact.
//  * O^T += V^T P: operand B is P, column c < G holding bf16(p) and column
//    G + c holding bf16(p - bf16(p)) of head c (so p too is split to ~2^-17);
//    the token order of its k slots is the order in which the S lanes hold
//    the scores, so P needs no shuffle. Operand A is V^T, which needs 8
//    tokens of one element per lane: the V tile is staged in LDS and read
//    with ds_read_b64_tr_b16. At the end column c + G is added to column c.
//  * Memory: each step's K and V loads are issued (16-byte non-temporal
//    loads, 16 KB per wavefront for D = 128) before the previous step is
//    consumed, into a second register set, so every wavefront keeps a step
//    in flight. V rows go to LDS after the products of the previous step
//    (a wavefront's LDS operations execute in order, so no barrier).
//  * Tiles are aligned to 16 tokens of the sequence, so a tile lies inside
//    one page (block_size >= 16) and its rows are one base plus a lane
//    offset. Tokens outside the piece are masked (score -inf); V rows past
//    the sequence's fill are zeroed, so uninitialised pool memory cannot
//    turn 0 * garbage into NaN. A fused append's token is taken from the
//    input in the step that holds it, rounded to bf16 and written to the
//    cache by the lanes that hold it.
// No atomics: results are bitwise reproducible, and a paged cache gives the
// bits of the same rows in a contiguous one.
#include "decode_kernels.h"

namespace skv {
namespace dec {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));

constexpr int kStep = 32;      // tokens per wavefront step (two 16-token tiles)
constexpr float kLazy = 8.f;   // rescale when the max grows by more than this (log2 units)
constexpr int kWaves = 8;      // wavefronts per workgroup

template <int D>
struct Gq {
  static constexpr int KB = D / 32;       // 32-element k-blocks of a K row
  static constexpr int CPR = D / 8;       // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;    // V rows per wavefront load
  static constexpr int VL = kStep / RPI;  // V loads per lane and step
  static constexpr int DB = D / 16;       // 16-row blocks of O^T
  // LDS bytes per V row: 32 bytes of padding put the rows of a transposed
  // read (8 rows x 2 chunks per half-wavefront) and of a row store (16 or
  // 8 chunks) on distinct banks.
  static constexpr int LROW = 2 * D + 32;
  static constexpr int TILE = kStep * LROW;  // a wavefront's V tile
};

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives as its slot
// j the element i%4 of the four 16-bit values addressed by lane 4j + i/4.
__device__ __forceinline__ i16x4 lds_read_tr16(const char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4*)(const_cast<char*>(p)));
}

// Eight elements of a runtime-dtype row, rounded to bf16 (round to nearest
// even), as four packed words.
__device__ __forceinline__ u32x4_t load8_bf16(const void* p, size_t i, int dt) {
  float x[8];
  load8_f32(p, i, dt, x);
  bf16x8 h;
#pragma unroll
  for (int j = 0; j < 8; ++j) h[j] = (__bf16)x[j];
  return __builtin_bit_cast(u32x4_t, h);
}

// A wavefront-uniform 32-bit value that no kernel of the call writes (the
// page table), read through the constant address space: a scalar load,
// waited for on its own counter. A plain load of it compiles to a vector
// load (the kernel's stores could alias it), and waiting for that vector
// load waited for every K/V load in flight as well.
__device__ __forceinline__ int load_uniform(const int32_t* p) {
  return *(const __attribute__((address_space(4))) int32_t*)(p);
}

template <int G>
__device__ __forceinline__ float shl_cols(float x) {  // lane i <- lane i + G of its 16-lane row
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x100 + G, 0xF, 0xF,
                                                    false));
}

// One piece [start, end) of sequence b for kv head group hg; the partials go
// to `slot`. smem: the workgroup's V tiles (kWaves * TILE bytes).
template <int D, int G, bool PAGED>
__device__ __forceinline__ void gqa_piece(const DecodeArgs& a, int hg, int b, int start, int end,
                                          int slot, char* smem) {
  using Sh = Gq<D>;
  constexpr int KB = Sh::KB, CPR = Sh::CPR, RPI = Sh::RPI, VL = Sh::VL, DB = Sh::DB;
  constexpr int LROW = Sh::LROW;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hw = a.hw, S = a.S;
  const int hl = wave % hw, sub = wave / hw;
  const int hk = hg * hw + hl;
  const int h = lane >> 4, c = lane & 15;
  const size_t RS = (size_t)a.Hkv * D;  // elements between consecutive tokens of a kv head
  char* vt = smem + wave * Sh::TILE;

  // ---- query operand: columns c and G + c hold head c % G; k-block kb < KB
  // takes q_hi, KB + kb takes q_lo, elements 32 kb + 8 h + j ----
  bf16x8 qf[2 * KB];
  {
    const bool used = c < 2 * G;
    const size_t qoff = ((size_t)b * a.Hq + hk * G + (used ? c % G : 0)) * D + 8 * h;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      float x[8];
      load8_f32(a.q, qoff + 32 * kb, a.q_dt, x);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float v = used ? x[j] * a.qscale : 0.f;
        const __bf16 hi = (__bf16)v;
        qf[kb][j] = hi;
        qf[KB + kb][j] = (__bf16)(v - (float)hi);
      }
    }
  }

  const bool has_new = appends(a, b) && end == clamped_len(a, b);
  const int mend = has_new ? end - 1 : end;  // the appended token's position, if any
  const int T0 = start & ~15;
  const int nsteps = (end - T0 + kStep - 1) / kStep;
  const int tlast = (end - 1) & ~15;  // the last tile holding a token of the piece
  const uint16_t* kc = static_cast<const uint16_t*>(a.k);
  const uint16_t* vc = static_cast<const uint16_t*>(a.v);

  // First element of the tile at token T (a multiple of 16, clamped to the
  // last tile of the piece so no page past the fill is looked up) for this
  // kv head. All 16 rows of a tile may be read: a page holds whole tiles
  // (block_size >= 16), and a contiguous cache whole ones too (T_cap % 16 ==
  // 0, checked by the dispatch). Uniform over the wavefront.
  auto tile_base = [&](int T) -> const uint16_t* {
    const int Tt = min(T, tlast);
    size_t row;
    if constexpr (PAGED) {
      const int blk = load_uniform(a.block_table + (size_t)b * a.max_blocks + (Tt >> a.bs_shift));
      row = ((size_t)blk << a.bs_shift) + (Tt & ((1 << a.bs_shift) - 1));
    } else {
      row = (size_t)b * a.T_cap + Tt;
    }
    return reinterpret_cast<const uint16_t*>(0) + (row * a.Hkv + hk) * D;
  };
  // lane offsets (elements) from a tile's first element: K operand rows and
  // V staging rows
  const uint32_t koff = (uint32_t)(c * RS + 8 * h);
  const uint32_t voff = (uint32_t)((lane / CPR) * RS + 8 * (lane % CPR));
  const size_t vstep = (size_t)RPI * RS;  // between the V loads of one lane
  auto at = [](const uint16_t* cache, const uint16_t* rel, size_t e) {
    return cache + (rel - reinterpret_cast<const uint16_t*>(0)) + e;
  };

  // Loads of step k: K rows into kr (MFMA operand layout), V rows into vr
  // (row u*RPI + lane/CPR of the step, chunk lane%CPR).
  auto issue_v = [&](int k, u32x4_t (&vr)[VL]) {
    const int T = T0 + k * kStep;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint16_t* base = tile_base(T + 16 * t);
#pragma unroll
      for (int u = 0; u < VL / 2; ++u)
        vr[t * VL / 2 + u] = stream_load16(at(vc, base, u * vstep) + voff);
    }
  };
  auto issue_k = [&](int k, u32x4_t (&kr)[2][KB]) {
    const int T = T0 + k * kStep;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint16_t* kp = at(kc, tile_base(T + 16 * t), koff);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) kr[t][kb] = stream_load16(kp + 32 * kb);
    }
  };

  // Step k's data has arrived: V rows past the sequence's fill are zeroed
  // (they may be uninitialised memory), then the rows go to LDS.
  auto finish = [&](int k, u32x4_t (&vr)[VL]) {
    const int T = T0 + k * kStep;
    if (T + kStep > end) {  // uniform: the step reaches past the piece
#pragma unroll
      for (int u = 0; u < VL; ++u)
        if (T + u * RPI + lane / CPR >= end) vr[u] = u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < VL; ++u)
      *reinterpret_cast<u32x4_t*>(vt + (u * RPI + lane / CPR) * LROW + 16 * (lane % CPR)) = vr[u];
  };

  // A fused append's token: the wavefront that reads the piece's last step
  // stores the input rows (rounded to bf16) at position mend first; before
  // it issues the loads of that step it waits for its stores to complete,
  // and then reads the row like any other.
  const bool writes_new = has_new && (nsteps - 1) % S == sub;
  if (writes_new) {
    const size_t nsrc = ((size_t)b * a.Hkv + hk) * D;
    const int tt = mend & ~15, ln = lane & (CPR - 1);
    const uint16_t* base = tile_base(tt);
    if (lane < 2 * CPR) {  // lanes [0, CPR): the K row, [CPR, 2 CPR): the V row
      const bool isv = lane >= CPR;
      const u32x4_t x = load8_bf16(isv ? a.new_v : a.new_k, nsrc + 8 * ln, a.in_dt);
      *reinterpret_cast<u32x4_t*>(const_cast<uint16_t*>(
          at(isv ? vc : kc, base, (size_t)(mend - tt) * RS + 8 * ln))) = x;
    }
  }

  f32x4 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  // transposed-read offset: lane c of group h addresses row 4h + c/4,
  // elements 4 (c%4) .. +3 of each 16-element block
  const int rd = (4 * h + (c >> 2)) * LROW + 8 * (c & 3);
  const float lo_f = c >= G ? 1.f : 0.f;

  // Scores of step k (K in kr): lane (h, c) gets column c at tokens
  // T + 4h + j (s[j]) and T + 16 + 4h + j (s[4 + j]), tokens outside the
  // piece masked.
  auto scores = [&](int k, const u32x4_t (&kr)[2][KB], float (&s)[8]) {
    const int T = T0 + k * kStep;
    f32x4 s0 = f32x4{0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
    for (int kb = 0; kb < 2 * KB; ++kb) {
      s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kr[0][kb % KB]),
                                                    qf[kb], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kr[1][kb % KB]),
                                                    qf[kb], s1, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s[j] = s0[j];
      s[4 + j] = s1[j];
    }
    if (T < start || T + kStep > end) {  // uniform
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int tok = T + (j >> 2) * 16 + 4 * h + (j & 3);
        if (tok < start || tok >= end) s[j] = -INFINITY;
      }
    }
  };

  // Online softmax and O^T update of step k (V in this wave's tile).
  auto consume = [&](float (&s)[8]) {
    float mt = s[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) mt = fmaxf(mt, s[j]);
    mt = fmaxf(mt, __shfl_xor(mt, 16));
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    // Lazy max: m moves only when some column's max passed it by more than
    // kLazy (uniform decision); the accumulator is then rescaled by al < 1,
    // else by 1 (a multiply in place: a branch around it made the compiler
    // copy every accumulator register).
    const float mn = __any(mt > m_run + kLazy) ? fmaxf(m_run, mt) : m_run;
    const float al = fast_exp2(m_run - mn);  // 0 on the first step, 1 if m stays
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] *= al;
    l_run *= al;
    m_run = mn;
    // P operand: bf16(p) in columns c < G, bf16(p - bf16(p)) in columns
    // G + c (y = p - lo_f * bf16(p), lo_f = 1 there, else 0); the columns
    // past 2G see q = 0, p = 1 and are never read.
    bf16x8 pf;
    float ls = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      const float p0 = fast_exp2(s[j] - m_run), p1 = fast_exp2(s[j + 1] - m_run);
      ls += p0 + p1;
      const bf16x2 hb = __builtin_convertvector(float2_t{p0, p1}, bf16x2);
      const uint32_t hw2 = __builtin_bit_cast(uint32_t, hb);
      const float y0 = fmaf(-lo_f, __uint_as_float(hw2 << 16), p0);
      const float y1 = fmaf(-lo_f, __uint_as_float(hw2 & 0xffff0000u), p1);
      const bf16x2 yb = __builtin_convertvector(float2_t{y0, y1}, bf16x2);
      pf[j] = yb[0];
      pf[j + 1] = yb[1];
    }
    l_run += ls;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const i16x4 v0 = lds_read_tr16(vt + rd + 32 * db);
      const i16x4 v1 = lds_read_tr16(vt + rd + 16 * LROW + 32 * db);
      const bf16x8 va =
          __builtin_bit_cast(bf16x8, __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
      o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pf, o[db], 0, 0, 0);
    }
  };

  // Pipeline over this wavefront's steps sub, sub + S, ...: step k + S is
  // loaded (K, then V) once step k's scores are formed, so its 16 KB (D =
  // 128) are in flight while step k is consumed; the only wait of a step is
  // for those loads, before its V rows go to LDS. (Issuing V of step k + S
  // before step k's scores left the compiler's wait counting unable to tell
  // the loop's registers from the prologue's: it waited on step k's K loads
  // before every V load.)
  {
    u32x4_t kr[2][KB], vr[VL];
    auto load_step = [&](int k) {
      if (writes_new && k == nsteps - 1) __builtin_amdgcn_s_waitcnt(0);  // appended rows stored
      issue_k(k, kr);
      issue_v(k, vr);
    };
    int k = sub;
    if (k < nsteps) {
      load_step(k);
      finish(k, vr);
    }
    for (; k < nsteps; k += S) {
      const int k2 = k + S;
      float s[8];
      scores(k, kr, s);
      if (k2 < nsteps) load_step(k2);
      consume(s);
      if (k2 < nsteps) finish(k2, vr);
    }
  }

  // ---- epilogue: l over the four lane groups; column G + c into column c ----
  float lt = l_run + __shfl_xor(l_run, 16);
  lt += __shfl_xor(lt, 32);
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int r = 0; r < 4; ++r) o[db][r] += shl_cols<G>(o[db][r]);
  // lane (h, c < G) holds head c's o at d = 16 db + 4 h + r

  if (S == 1) {
    if (c < G) {
      const size_t pidx = (size_t)(hk * G + c) * a.n_slots + slot;
#pragma unroll
      for (int db = 0; db < DB; ++db)
        *reinterpret_cast<f32x4*>(a.ws_o + pidx * D + 16 * db + 4 * h) = o[db];
      if (h == 0) *reinterpret_cast<float2*>(a.ws_ml + pidx * 2) = make_float2(m_run, lt);
    }
    return;
  }

  // S > 1: the S substreams of each kv head merge through LDS (the V tiles'
  // space). Substreams that saw no step drop out through exp2(-inf) = 0.
  float* mo = reinterpret_cast<float*>(smem);         // [kWaves][G][D]
  float* mml = mo + kWaves * G * D;                   // [kWaves][G][2]
  __syncthreads();  // every wavefront is done with its tile
  if (c < G) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
      *reinterpret_cast<f32x4*>(mo + (wave * G + c) * D + 16 * db + 4 * h) = o[db];
    if (h == 0) {
      mml[(wave * G + c) * 2 + 0] = m_run;
      mml[(wave * G + c) * 2 + 1] = lt;
    }
  }
  __syncthreads();
  for (int idx = tid; idx < hw * G * D; idx += kWaves * 64) {
    const int hh = idx / (G * D), g = (idx / D) % G, d = idx % D;
    float M = -INFINITY;
    for (int s2 = 0; s2 < S; ++s2) M = fmaxf(M, mml[((hh + s2 * hw) * G + g) * 2]);
    float L = 0.f, O = 0.f;
    for (int s2 = 0; s2 < S; ++s2) {
      const int wv = hh + s2 * hw;
      const float wgt = fast_exp2(mml[(wv * G + g) * 2] - M);
      L = fmaf(wgt, mml[(wv * G + g) * 2 + 1], L);
      O = fmaf(wgt, mo[(wv * G + g) * D + d], O);
    }
    const size_t pidx = (size_t)((hg * hw + hh) * G + g) * a.n_slots + slot;
    a.ws_o[pidx * D + d] = O;
    if (d == 0) *reinterpret_cast<float2*>(a.ws_ml + pidx * 2) = make_float2(M, L);
  }
  __syncthreads();  // the next piece's V tiles overwrite this space
}

// Grid (n_wg, H_kv / hw), kWaves wavefronts: wavefront w serves kv head
// w % hw of the group and token substream w / hw.
template <int D, int G, bool PAGED>
__global__ __launch_bounds__(kWaves * 64) void k_decode_gqa(DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[kWaves * Gq<D>::TILE];
  static_assert(kWaves * Gq<D>::TILE >= kWaves * 8 * D * 4 + kWaves * 8 * 2 * 4,
                "the substream merge reuses the V tiles' space");
  const int w = blockIdx.x, hg = blockIdx.y;
  int b, off;
  locate(a, (long long)w * a.chunk, w == 0 && hg == 0, &b, &off);
  if (b < 0) return;  // uniform over the workgroup
  int budget = a.chunk;
  while (true) {
    const int n = min(clamped_len(a, b) - off, budget);
    gqa_piece<D, G, PAGED>(a, hg, b, off, off + n, w + b, smem);
    budget -= n;
    if (budget == 0) break;
    do {
      ++b;
    } while (b < a.B && clamped_len(a, b) == 0);
    if (b >= a.B) break;
    off = 0;
  }
}

template <int D, int G>
void launch_dg(const DecodeArgs& a, bool paged, hipStream_t s) {
  const dim3 grid(a.n_wg, a.Hkv / a.hw);
  if (paged) hipLaunchKernelGGL((k_decode_gqa<D, G, true>), grid, dim3(kWaves * 64), 0, s, a);
  else hipLaunchKernelGGL((k_decode_gqa<D, G, false>), grid, dim3(kWaves * 64), 0, s, a);
}

}  // namespace

bool gqa_mfma_eligible(const DecodeArgs& a, int G, bool bf16_cache, bool paged) {
  return bf16_cache && (a.D == 64 || a.D == 128) && (G == 2 || G == 4 || G == 8) &&
         (paged ? a.bs_shift >= 4 : a.T_cap % 16 == 0);
}

int launch_partial_gqa(const DecodeArgs& a0, int G, bool paged, hipStream_t s) {
  DecodeArgs a = a0;
  // kv heads per workgroup: the largest power of two <= kWaves dividing H_kv;
  // the remaining wavefronts split each head's tokens into substreams
  a.hw = 1;
  while (a.hw < kWaves && a.Hkv % (a.hw * 2) == 0) a.hw *= 2;
  a.S = kWaves / a.hw;
  if (a.Hkv / a.hw > 65535)
    return set_error(SKV_E_UNSUPPORTED, "skv_decode_attn: H_kv=%d exceeds the grid limit", a.Hkv);
#define SKV_GQ(DD, GG)               \
  if (a.D == DD && G == GG) {        \
    launch_dg<DD, GG>(a, paged, s);  \
    return 0;                        \
  }
  SKV_GQ(128, 4) SKV_GQ(128, 2) SKV_GQ(128, 8) SKV_GQ(64, 4) SKV_GQ(64, 2) SKV_GQ(64, 8)
#undef SKV_GQ
  return set_error(SKV_E_UNSUPPORTED, "skv_decode_attn: no MFMA kernel for head_dim %d, G=%d",
                   a.D, G);
}

}  // namespace dec
}  // namespace skv
