// Pass 1 of cached decode attention with grouped queries on the matrix
// cores: bf16 caches, head dim 64 or 128, G = H_q / H_kv in {2, 4, 8}.
//
// Same work split, partial format and merge pass as the VALU kernels
// (decode_kernels.h): workgroup w owns tokens [w*chunk, (w+1)*chunk) of the
// flat token stream, cut into pieces at sequence boundaries, and writes one
// partial (m, l, o[D]) per (piece, query head) at slot w + b. What differs is
// how a piece is consumed. With G query heads per kv head the VALU kernels
// spend ~36 wavefront instructions per (token, kv head) on the q.k dots, the
// p.V updates and their cross-lane sums; here both products run on MFMA and
// the VALU is left with the softmax itself (~4 instructions per token and
// kv head), so the pass is bound by HBM.
//
// Memory: a workgroup of 8 wavefronts serves hw kv heads (hw = 8 for C5's
// 8 kv heads) and moves its tokens through LDS in stages of 16*S tokens x hw
// heads, K then V (S = 8 / hw token substreams; 32 KB per tensor at D =
// 128). The cache rows of consecutive heads of a token are adjacent, so a
// stage is read as contiguous 1 KB pieces (16-byte non-temporal loads),
// two stages in flight in registers while the previous one is consumed
// from LDS. (A first form
// in which each wavefront read only its own head's 256-byte rows, 2 KB
// apart, streamed at 65% of 8 TB/s on C5; the VALU kernels, which read 1 KB
// contiguous per instruction, reach 85% on C4.) Each 16-byte chunk of a row
// is stored at position chunk ^ swz(token), which puts both read patterns
// below on distinct LDS banks.
//
// Compute: wavefront (hl, sub) takes kv head hl and tokens [16 sub, 16 sub
// + 16) of each stage, for its G query heads:
//  * S = K q^T (v_mfma_f32_16x16x32_bf16): operand A is the K tile (lane l
//    holds row l%16, 8 elements per k-block), operand B the query: column
//    c < G holds head c, column G + c head c again, and the k dimension is
//    [D elements of q_hi ; D elements of q_lo], q_hi = bf16(q * scale *
//    log2 e), q_lo = bf16(that - q_hi), against [K | K]. The split makes q.k
//    exact to ~2^-17 relative (K is bf16 already); the duplicated columns
//    give columns c and G + c the same score, bit for bit.
//  * Online softmax per column, each lane holding 4 of the 16 scores. The
//    running max moves lazily: only when a stage's max passes it by more
//    than 8 (log2 units), so p = exp2(s - m) <= 256; (m, l, o) stay
//    consistent and the merge is exact.
//  * O^T += V^T P (v_mfma_f32_16x16x16_bf16): operand B is P, column c < G
//    holding bf16(p) and column G + c bf16(p - bf16(p)) of head c, in the
//    token order in which the score lanes hold them (no shuffle); operand A
//    is V^T, 4 tokens of one element per lane, read with ds_read_b64_tr_b16.
//    At the end column G + c is added to column c.
// Tokens outside the piece are masked (score -inf), and their rows are
// loaded from its first or last row: no page past the fill is touched, no
// uninitialised memory meets a zero weight (0 * NaN), and the first tile's
// tokens before the piece (another workgroup's) cost no HBM traffic. A fused append's rows
// are stored to the cache (rounded to bf16) at the start of the piece, and
// the stores complete before any wavefront loads the stage holding them.
// No atomics: results are bitwise reproducible, and a paged cache gives the
// bits of the same rows in a contiguous one.
#include "decode_kernels.h"

namespace skv {
namespace dec {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;     // wavefronts per workgroup
constexpr int kSub = 16;      // tokens per wavefront and stage (one MFMA tile)
constexpr float kLazy = 8.f;  // rescale when the max grows by more than this (log2 units)
constexpr int kMaxChunk = 8192;                // longest chunk (tokens) the kernel takes
constexpr int kMaxTiles = kMaxChunk / 16 + 2;  // 16-token tiles a piece can touch

template <int D>
struct Gq {
  static constexpr int KB = D / 32;   // 32-element k-blocks of a K row
  static constexpr int CPR = D / 8;   // 16-byte chunks per row
  static constexpr int DB = D / 16;   // 16-row blocks of O^T
  static constexpr int TBYTES = kWaves * kSub * D * 2;  // one tensor's rows of a stage
  static constexpr int SBYTES = 2 * TBYTES;             // a stage: K, then V
  static constexpr int NI = TBYTES / (kWaves * 1024);   // 1 KB pieces per wavefront and tensor
};

// Physical 16-byte chunk position of logical chunk lc in the row of stage
// token t is lc ^ swz(t). At D = 128 (a row is the 256 bytes of one bank
// sweep): the K operand reads take one chunk of 16 consecutive tokens'
// rows (swz injective on t % 16), the transposed V reads two adjacent
// chunks of 8 consecutive tokens' rows (swz / 2 injective on t % 8).
template <int D>
__device__ __forceinline__ int swz(int t) {
  return (2 * (t & 7) + ((t >> 3) & 1)) & (D / 8 - 1);
}

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

template <int G>
__device__ __forceinline__ float shl_cols(float x) {  // lane i <- lane i + G of its 16-lane row
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x100 + G, 0xF, 0xF,
                                                    false));
}

// One piece [start, end) of sequence b for kv head group hg; the partials go
// to `slot`. smem: one stage (SBYTES bytes); s_rows: kMaxTiles cache rows.
template <int D, int G, bool PAGED>
__device__ __forceinline__ void gqa_piece(const DecodeArgs& a, int hg, int b, int start, int end,
                                          int slot, char* smem, long long* s_rows) {
  using Sh = Gq<D>;
  constexpr int KB = Sh::KB, CPR = Sh::CPR, DB = Sh::DB, NI = Sh::NI;
  constexpr int TBYTES = Sh::TBYTES;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hw = a.hw, S = a.S;  // hw * S == kWaves, both powers of two
  const int lhw = __builtin_ctz(hw);
  const int hl = wave & (hw - 1), sub = wave >> lhw;
  const int hk = hg * hw + hl;
  const int h = lane >> 4, c = lane & 15;
  const int TS = kSub * S;  // tokens per stage

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
  const int nst = (end - T0 + TS - 1) / TS;
  const int tlast = (end - 1) & ~15;  // the last 16-token tile holding a token of the piece
  const uint16_t* kc = static_cast<const uint16_t*>(a.k);
  const uint16_t* vc = static_cast<const uint16_t*>(a.v);

  // Cache rows of the piece's 16-token tiles. Paged: looked up once per
  // piece into LDS (one vector load per tile, all in flight together), so a
  // stage's loads do not wait on a page-table read.
  if constexpr (PAGED) {
    const int ntiles = (tlast - T0) / 16 + 1;
    for (int i = tid; i < ntiles; i += kWaves * 64) {
      const int Tt = T0 + 16 * i;
      const long long blk = a.block_table[(size_t)b * a.max_blocks + (Tt >> a.bs_shift)];
      s_rows[i] = (blk << a.bs_shift) + (Tt & ((1 << a.bs_shift) - 1));
    }
    __syncthreads();
  }
  // Cache row of token Tt (a multiple of 16, in [T0, tlast]); uniform.
  auto tile_row = [&](int Tt) -> size_t {
    if constexpr (PAGED) {
      const long long r = s_rows[(Tt - T0) >> 4];  // the same for every lane
      const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)r);
      const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(r >> 32));
      return ((size_t)hi << 32) | lo;
    } else {
      return (size_t)b * a.T_cap + Tt;
    }
  };

  // A fused append: the rows of the group's hw heads go to position mend,
  // stored by threads [0, 2 hw CPR) (K, then V), before any load.
  if (has_new) {
    const int nrow = hw * CPR;
    if (tid < 2 * nrow) {
      const bool isv = tid >= nrow;
      const int u = isv ? tid - nrow : tid, hd = u / CPR, ln = u % CPR;
      const size_t src = ((size_t)b * a.Hkv + hg * hw + hd) * D + 8 * ln;
      const u32x4_t x = load8_bf16(isv ? a.new_v : a.new_k, src, a.in_dt);
      const size_t row = tile_row(mend & ~15) + (mend & 15);
      uint16_t* dst = const_cast<uint16_t*>(isv ? vc : kc) + (row * a.Hkv + hg * hw + hd) * D;
      *reinterpret_cast<u32x4_t*>(dst + 8 * ln) = x;
    }
    __builtin_amdgcn_s_waitcnt(0);  // the stores have completed
    __syncthreads();
  }

  // Loads of stage k (tokens [T0 + k TS, + TS)) into r: the 16-byte unit
  // pos of a tensor's stage rows is row pos / CPR = t * hw + hd (stage
  // token t, head hd of the group), physical chunk pos % CPR; wavefront w
  // moves the 1 KB pieces [w NI, (w + 1) NI) of K (r[i]) and of V
  // (r[NI + i]). A piece's rows lie in one 16-token tile (a piece holds 1
  // to 8 whole tokens), so its page is uniform. Rows outside the piece
  // are read from its first or last row.
  // A wavefront's pieces hold stage tokens [2 S w, 2 S w + 2 S) (16 / hw
  // tokens per 2 D units), all in one 16-token tile.
  const int twave = (wave * NI * 64 / CPR) >> lhw;
  auto load_stage = [&](int k, u32x4_t (&r)[2 * NI]) {
    const int T = T0 + k * TS;
    const int Tt = min(T + (twave & ~15), tlast);
    const size_t trow = tile_row(Tt);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int piece = wave * NI + i;
      const int pos = piece * 64 + lane;
      const int ri = pos / CPR;
      const int t = ri >> lhw, hd = ri & (hw - 1);
      const int lc = (pos % CPR) ^ swz<D>(t);
      // rows outside the piece (the first tile's tokens before start, the
      // last one's past end) reread the piece's first or last row: masked
      // anyway, and an L2 hit instead of a fetch from HBM
      const int tok = min(max(T + t, start), end - 1);
      const size_t e = ((trow + (tok - Tt)) * a.Hkv + hg * hw + hd) * D + 8 * lc;
      r[i] = stream_load16(kc + e);
      r[NI + i] = stream_load16(vc + e);
    }
  };
  // ... and into the LDS stage, at unit pos
  auto store_stage = [&](const u32x4_t (&r)[2 * NI]) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      char* p = smem + (wave * NI + i) * 1024 + 16 * lane;
      *reinterpret_cast<u32x4_t*>(p) = r[i];
      *reinterpret_cast<u32x4_t*>(p + TBYTES) = r[NI + i];
    }
  };

  // LDS offsets (within a stage) of this lane's operand reads: the K rows
  // of stage token 16 sub + c, chunk 4 kb + h; the V rows of stage token
  // 16 sub + 4h + c/4, elements 16 db + 4 (c%4) .. + 3.
  int kaddr[KB], vaddr[DB];
  {
    const int tk = kSub * sub + c;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
      kaddr[kb] = ((tk * hw + hl) * CPR + ((4 * kb + h) ^ swz<D>(tk))) * 16;
    const int tv = kSub * sub + 4 * h + (c >> 2);
#pragma unroll
    for (int db = 0; db < DB; ++db)
      vaddr[db] = TBYTES + ((tv * hw + hl) * CPR + ((2 * db + ((c & 3) >> 1)) ^ swz<D>(tv))) * 16 +
                  8 * (c & 1);
  }

  f32x4 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  const float lo_f = c >= G ? 1.f : 0.f;

  // This wavefront's 16 tokens of stage k, from the LDS stage.
  auto compute = [&](int k) {
    const int T = T0 + k * TS + kSub * sub;  // first token of this wavefront's tile
    if (T >= end) return;                    // uniform: a tile past the piece is idle
    const char* st = smem;
    bf16x8 kf[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) kf[kb] = *reinterpret_cast<const bf16x8*>(st + kaddr[kb]);
    f32x4 sc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 2 * KB; ++kb)
      sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[kb % KB], qf[kb], sc, 0, 0, 0);
    // lane (h, c) holds column c at tokens T + 4h + j
    float s[4] = {sc[0], sc[1], sc[2], sc[3]};
    if (T < start || T + kSub > end) {  // uniform
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tok = T + 4 * h + j;
        if (tok < start || tok >= end) s[j] = -INFINITY;
      }
    }
    float mt = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    mt = fmaxf(mt, __shfl_xor(mt, 16));
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    // Lazy max: m moves only when some column's max passed it by more than
    // kLazy (uniform decision); the accumulator is then rescaled by al < 1,
    // else by 1 (a multiply in place: a branch around it made the compiler
    // copy every accumulator register).
    const float mn = __any(mt > m_run + kLazy) ? fmaxf(m_run, mt) : m_run;
    const float al = fast_exp2(m_run - mn);  // 0 on the first tile, 1 if m stays
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] *= al;
    l_run *= al;
    m_run = mn;
    // P operand: bf16(p) in columns c < G, bf16(p - bf16(p)) in columns
    // G + c (y = p - lo_f * bf16(p), lo_f = 1 there, else 0); the columns
    // past 2G see q = 0, p = 1 and are never read.
    i16x4 pf;
    float ls = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j += 2) {
      const float p0 = fast_exp2(s[j] - m_run), p1 = fast_exp2(s[j + 1] - m_run);
      ls += p0 + p1;
      const uint32_t hb =
          __builtin_bit_cast(uint32_t, __builtin_convertvector(float2_t{p0, p1}, bf16x2));
      const float y0 = fmaf(-lo_f, __uint_as_float(hb << 16), p0);
      const float y1 = fmaf(-lo_f, __uint_as_float(hb & 0xffff0000u), p1);
      const uint32_t yb =
          __builtin_bit_cast(uint32_t, __builtin_convertvector(float2_t{y0, y1}, bf16x2));
      pf[j] = (short)(yb & 0xffffu);
      pf[j + 1] = (short)(yb >> 16);
    }
    l_run += ls;
#pragma unroll
    for (int db = 0; db < DB; ++db)
      o[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(lds_read_tr16(st + vaddr[db]), pf, o[db],
                                                         0, 0, 0);
  };

  // Two stages in flight, in two register sets: stages k + 1 and k + 2 are
  // loading while stage k is consumed from LDS; then stage k + 1 goes to
  // LDS and stage k + 3 is issued into the set it leaves. (Loads straight
  // into LDS need no registers, but the compiler cannot tell which LDS a
  // pending one writes and waited for all of them before the first LDS
  // read of every stage.) The steady-state loop issues its loads without
  // conditions: the compiler counts outstanding loads per path, and a load
  // behind a branch made it wait for both sets before every LDS store.
  {
    u32x4_t ra[2 * NI], rb[2 * NI];
    if (nst > 4) {
      load_stage(0, ra);
      load_stage(1, rb);
      store_stage(ra);
      __syncthreads();
      load_stage(2, ra);
      int k = 0;
      for (; k + 4 < nst; k += 2) {  // stages k + 1 (rb), k + 2 (ra) in flight
        compute(k);
        __syncthreads();  // every wavefront is done with stage k
        store_stage(rb);
        __syncthreads();
        load_stage(k + 3, rb);
        compute(k + 1);
        __syncthreads();
        store_stage(ra);
        __syncthreads();
        load_stage(k + 4, ra);
      }
      // stages k (LDS), k + 1 (rb), k + 2 (ra) and perhaps k + 3 are left
      const bool four = k + 3 < nst;
      compute(k);
      __syncthreads();
      store_stage(rb);
      __syncthreads();
      if (four) load_stage(k + 3, rb);
      compute(k + 1);
      __syncthreads();
      store_stage(ra);
      __syncthreads();
      compute(k + 2);
      if (four) {
        __syncthreads();
        store_stage(rb);
        __syncthreads();
        compute(k + 3);
      }
    } else {  // a short piece: up to 4 stages
      load_stage(0, ra);
      if (nst > 1) load_stage(1, rb);
      store_stage(ra);
      __syncthreads();
      compute(0);
      if (nst > 1) {
        if (nst > 2) load_stage(2, ra);
        __syncthreads();
        store_stage(rb);
        __syncthreads();
        compute(1);
        if (nst > 2) {
          if (nst > 3) load_stage(3, rb);
          __syncthreads();
          store_stage(ra);
          __syncthreads();
          compute(2);
          if (nst > 3) {
            __syncthreads();
            store_stage(rb);
            __syncthreads();
            compute(3);
          }
        }
      }
    }
    __syncthreads();  // the stage's space is free for the merge or the next piece
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

  // S > 1: the S substreams of each kv head merge through LDS (the stage's
  // space: every wavefront is past the loop's last barrier). Substreams
  // that saw no token drop out through exp2(-inf) = 0.
  float* mo = reinterpret_cast<float*>(smem);  // [kWaves][G][D]
  float* mml = mo + kWaves * G * D;            // [kWaves][G][2]
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
  __syncthreads();  // the next piece's stages overwrite this space
}

// Grid (n_wg, H_kv / hw), kWaves wavefronts: wavefront w serves kv head
// w % hw of the group and token substream w / hw.
template <int D, int G, bool PAGED>
__global__ __launch_bounds__(kWaves * 64) void k_decode_gqa(DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[Gq<D>::SBYTES];
  __shared__ long long s_rows[PAGED ? kMaxTiles : 1];
  static_assert(Gq<D>::SBYTES >= kWaves * 8 * D * 4 + kWaves * 8 * 2 * 4,
                "the substream merge reuses the stage's space");
  const int w = blockIdx.x, hg = blockIdx.y;
  int b, off;
  locate(a, (long long)w * a.chunk, w == 0 && hg == 0, &b, &off);
  if (b < 0) return;  // uniform over the workgroup
  int budget = a.chunk;
  while (true) {
    const int n = min(clamped_len(a, b) - off, budget);
    gqa_piece<D, G, PAGED>(a, hg, b, off, off + n, w + b, smem, s_rows);
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
         (!paged || a.bs_shift >= 4) && a.chunk <= kMaxChunk;
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
