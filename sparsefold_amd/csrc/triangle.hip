// Triangle attention module (starting / ending node) on gfx950.
//
// Replaces GridSelfAttention.forward (src/sparsefold/model/trunk/blocks.py:293-366 with the
// per-chunk _attention of :270-291).
//
// Fast path (head dim 32, the trunk's C=128 / H=4 configuration):
//   0. tri_fold_kernel   folds the LN gamma into the packed projection weight and beta into
//                        a per-column offset (blocks.py:317 followed by :276-278, :286, :320).
//   1. tri_proj_kernel   persistent workgroups with the folded [Wq|Wk|Wv|Wg|Wb] resident in
//                        LDS; each wave normalises 32 positions of an attention row straight
//                        into MFMA operand registers and runs the projections, storing every
//                        operand head-major in the register order the attention MFMAs use, so
//                        that each store instruction writes 1 KB of contiguous memory:
//                          Q, K, G  per (row r, head h), 32-position blocks of
//                                   [k-chunk 2][lane half 2][position 32][8 dims]; q carries
//                                   scale * log2(e), so logits land in log2 units
//                          V^T      per (row r, head h), 16-key chunks of
//                                   [lane half 2][dim 32][8 keys in PV slot order]
//                          bias     per (h, 32 queries, 64 keys) 4 KB blocks in the attention
//                                   loads' order (bias_off), bias * log2(e), bf16, untransposed orientation
//                                   (blocks.py:329), masked keys = SF_MASKED_LOGIT, keys past
//                                   N = -inf, keys in S^T register order
//                        For the ending node the workgroup walks z's column instead of its row,
//                        so nothing is transposed in memory (blocks.py:345-346, :362-363).
//   2. tri_attn_kernel   one workgroup per (4 rows, head, 256 queries); K / V^T tiles of 64
//                        keys for the 4 rows double-buffered in LDS; each wave keeps the
//                        softmax sums of its 32 queries for all 4 rows and feeds its bias tile
//                        -- identical for every row, loaded a tile ahead into its registers --
//                        as the accumulator input of the S^T MFMA;
//                        output written at its pair position, rows with an out-of-range
//                        weight sum flagged.
//      tri_fixup_kernel  rows whose token is masked attend uniformly to every key (the
//                        reference's finite -finfo.max mask): mean of V; flagged rows are
//                        recomputed with an exact two-pass softmax.
//   3. tri_out_kernel    out = z + o W_o (blocks.py:291, :366), W_o resident in LDS.
// Other head dims use the generic kernels (layer_norm, linear, attention_fwd, linear).
#include <cmath>
#include <type_traits>

#include "sf_common.h"

namespace {
size_t round_up(size_t x) { return (x + 255) & ~(size_t)255; }
// Padded token count of the fast path's operand layouts: a whole number of pairs of 64-key tiles,
// so that the attention kernel's double-buffered tile pipeline starts every task in buffer 0.
int round_np(int n) { return (n + 127) & ~127; }

// ---------------------------------------------------------------------------------------
// Operand layouts.
// S^T register order: lane half h', register a -> key 8*(a/4) + 4*h' + a%4 of a 32-key half.
__host__ __device__ inline int bias_pos64(int j) {
  const int j32 = j & 31;
  return (j & 32) + 16 * ((j32 >> 2) & 1) + 4 * (j32 >> 3) + (j32 & 3);
}
// Bias planes of the head-dim-32 path, in the order the attention kernel loads them: per (head h,
// tile of 32 queries, tile of 64 keys) one 4 KB block [piece k 4][lane 64][8 keys], where lane
// 32 h' + i%32 holds, as piece k, stored piece 4(k/2) + 2h' + k%2 (8 keys) of query i's 64 keys
// in stored (bias_pos64) order -- the keys its S^T registers hold.  Each of a wave's four
// 16-byte loads then reads 1 KB of contiguous memory: with a query row per lane (32 rows, each
// read in 16-byte pieces) the same loads ran at a third of the L2 bandwidth.
// js = stored key position in the row: (j & ~63) + bias_pos64(j & 63).
__host__ __device__ inline int64_t bias_off_stored(int h, int i, int js, int NP) {
  const int jp = js & 63, pc = jp >> 3;
  const int k = 2 * (pc >> 2) + (pc & 1), hf = (pc >> 1) & 1;
  return ((((int64_t)h * (NP >> 5) + (i >> 5)) * (NP >> 6) + (js >> 6)) << 11)
         + ((k * 64 + 32 * hf + (i & 31)) << 3) + (jp & 7);
}
__host__ __device__ inline int64_t bias_off(int h, int i, int j, int NP) {
  return bias_off_stored(h, i, (j & ~63) + bias_pos64(j & 63), NP);
}
// The operand layouts below are written for KC = D / 16 k-chunks of 16 dims per head: KC = 2 for
// head dim 32 (C = 128), KC = 1 for head dim 16 (C = 64).
// Attention output o of (head h, attention row r, query i): per (h, r, block of 32 queries) a
// block of KC KB [piece 2 KC][query 32][8 dims], piece KC hf + kk holding the 8 dims the attention
// epilogue's lane half hf stores as its k-chunk kk (dims 16 kk + 8 (t/4) + 4 hf + t%4 of the
// head, t = 0..7).  Each store
// of the epilogue (a piece of 32 queries per lane half) and each load of the output stage (a
// piece of 32 positions) then covers 512 contiguous bytes; with a query's 64 bytes contiguous,
// consecutive lanes were 64 bytes apart.  Indexed by attention row and query, not by pair
// position, so both nodes write whole blocks.
template <int KC = 2>
__host__ __device__ inline int64_t o_off(int h, int r, int i, int hf, int kk, int N, int NP) {
  return ((((int64_t)h * N + r) * (NP >> 5) + (i >> 5)) * (512 * KC)) + ((((KC * hf + kk) << 5) + (i & 31)) << 3);
}
// Q / K / G of (row r, head h): position p, k-chunk kk, lane half hf.  The 8 values at the
// returned offset are dims 16*kk + 8*(t/4) + 4*hf + t%4 for t = 0..7 -- what lane (p%32, hf)
// of a 32x32x16 MFMA holds for k-chunk kk, both as the A operand of S^T = K Q^T and, for Q,
// as its B operand, and what the D^T accumulator of the projection holds in registers
// 8*kk .. 8*kk+7.  The dot product q.k is invariant under this common dim permutation.
template <int KC = 2>
__host__ __device__ __forceinline__ int64_t ql_off(int r, int h, int H, int NP, int p, int kk, int hf) {
  return ((((int64_t)r * H + h) * (NP >> 5) + (p >> 5)) * (2 * KC) + kk * 2 + hf) * 256 + (p & 31) * 8;
}
// V^T of (row r, head h): 16-key chunk c16, lane half hf, dim d < 16 KC.  The 8 values are keys
// 16*c16 + 8*(t/4) + 4*hf + t%4 (PV slot order: the keys whose weights lane half hf holds).
template <int KC = 2>
__host__ __device__ __forceinline__ int64_t vl_off(int r, int h, int H, int NP, int c16, int hf, int d) {
  return ((((int64_t)r * H + h) * (NP >> 4) + c16) * 2 + hf) * (128 * KC) + d * 8;
}

// Sizes of the fast paths: KC = 2 (C = 128, head dim 32) and KC = 1 (C = 64, head dim 16), four
// heads each.
template <int KC>
struct TriDims {
  static constexpr int C = 64 * KC;                   // channels
  static constexpr int D = 16 * KC;                   // head dim
  static constexpr int WP = C + 8;                    // LDS pitch (elements) of weight rows
  static constexpr int NC = C / 16;                   // 16-channel k-chunks of a position
  static constexpr int NB = C / 32;                   // blocks of 32 rows of each of W_q, W_k, W_v, W_g, W_o
  static constexpr int Cols = (4 * NB + 1) * 32;      // folded rows: q k v g + bias block (32, 4 used)
  // Blocks of 32 folded rows the projection keeps in LDS: q (0 .. NB-1), k, v and the bias block
  // (folded block 4 NB, stored as LDS block 3 NB); the gate rows are used by the output kernel.
  static constexpr int ProjBlocks = 3 * NB + 1;
};
constexpr int kPC = 128;              // channels (C) of the head-dim-32 path
constexpr int kWP = kPC + 8;          // LDS pitch (elements) of weight rows
constexpr int kPWaves = 8;            // waves per projection / output workgroup

struct FastWs {
  uint16_t *q, *k, *vt, *bias, *o, *wf;
  float* off;
  uint8_t* flags;                     // [N][H] rows for the exact fix-up
  int* ctr;                           // fused epilogue: [G] per (row group, query block) heads done, then
                                      // the error word (see TriAttnArgs)
  uint8_t* defer;                     // [N] rows whose output the post kernel writes
  int* rgl;                           // [1 + NP/4]: count, then the row groups with a valid row
  int nctr;                           // G + 4
  size_t bytes;
};

// Groups of the fused epilogue: (row group of 4 rows, block of 256 queries).
int fused_groups(int32_t N) {
  const int NP = round_np(N);
  return (NP / 4) * ((NP + 255) / 256);
}

template <int KC = 2>
FastWs carve_fast(void* base, int32_t N, int32_t H) {
  using TD = TriDims<KC>;
  const size_t NP = (size_t)round_np(N), E = NP * NP * H * TD::D;
  FastWs w{};
  char* p = (char*)base;
  size_t off = 0;
  w.q = (uint16_t*)(p + off); off += round_up(E * 2);
  w.k = (uint16_t*)(p + off); off += round_up(E * 2);
  w.vt = (uint16_t*)(p + off); off += round_up(E * 2);
  w.bias = (uint16_t*)(p + off); off += round_up(NP * NP * H * 2);
  w.o = (uint16_t*)(p + off); off += round_up((size_t)N * NP * H * TD::D * 2);   // o_off blocks
  w.wf = (uint16_t*)(p + off); off += round_up((size_t)TD::Cols * TD::C * 2);
  w.off = (float*)(p + off); off += round_up((size_t)TD::Cols * 4);
  w.flags = (uint8_t*)(p + off); off += round_up((size_t)N * H);
  w.nctr = fused_groups(N) + 4;
  w.ctr = (int*)(p + off); off += round_up((size_t)w.nctr * 4);
  w.defer = (uint8_t*)(p + off); off += round_up((size_t)N);
  w.rgl = (int*)(p + off); off += round_up((size_t)(1 + NP / 4) * 4);
  w.bytes = off;
  return w;
}

// ---------------------------------------------------------------------------------------
// 0. weight fold: wf[n][c] = bf16(w[n][c] * gamma[c]), off[n] = sum_c beta[c] w[n][c];
//    rows 4 H D + H .. Cols-1 (padding of the bias block) are zero.  One wave per weight row.  Also clears
//    the attention kernel's fix-up flags.
// ---------------------------------------------------------------------------------------
struct TriFoldArgs {
  int nrows;                          // 4 * H * D + H
  const uint16_t* w;                  // [nrows, C]
  const float* ln_w; const float* ln_b;
  uint16_t* wf; float* off;           // [Cols, C], [Cols]
  uint8_t* flags; int nflags;         // [N * H], cleared
  int* ctr; int nctr;                 // fused epilogue counters, cleared
  uint8_t* defer; int ndefer;         // fused epilogue deferred rows, cleared
  // the attention rows worth computing: row groups (4 rows) with a row r < N and seq[r] != 0,
  // listed in rgl[1..count], count in rgl[0] (null: no list)
  int* rgl; int rg, N; const uint8_t* seq;
};

template <int KC>
__global__ __launch_bounds__(256) void tri_fold_kernel(const TriFoldArgs a) {
  using TD = TriDims<KC>;
  const int lane = threadIdx.x & 63;
  if (blockIdx.x == gridDim.x - 1) {                       // the extra last workgroup compacts the row groups
    if (a.rgl == nullptr) return;
    __shared__ int part[256];
    const int tid = threadIdx.x, per_t = (a.rg + 255) / 256;
    const int g0 = min(tid * per_t, a.rg), g1 = min(g0 + per_t, a.rg);
    auto valid = [&](int g) {
      bool v = false;
      for (int r = 4 * g; r < 4 * g + 4 && r < a.N; ++r) v |= a.seq[r] != 0;
      return v;
    };
    int cnt = 0;
    for (int g = g0; g < g1; ++g) cnt += valid(g);
    int inc = cnt;                                         // inclusive prefix within the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(inc, o);
      if (lane >= o) inc += v;
    }
    if (lane == 63) part[tid >> 6] = inc;                  // wave totals
    __syncthreads();
    int base = inc - cnt;                                  // exclusive prefix of the counts
    for (int w = 0; w < (tid >> 6); ++w) base += part[w];
    for (int g = g0; g < g1; ++g)
      if (valid(g)) a.rgl[1 + base++] = g;
    if (tid == 255) a.rgl[0] = base;
    return;
  }
  const int zstride = (gridDim.x - 1) * blockDim.x;         // the folding workgroups clear the flags
  for (int f = blockIdx.x * blockDim.x + threadIdx.x; f < a.nflags; f += zstride) a.flags[f] = 0;
  for (int f = blockIdx.x * blockDim.x + threadIdx.x; f < a.nctr; f += zstride) a.ctr[f] = 0;
  for (int f = blockIdx.x * blockDim.x + threadIdx.x; f < a.ndefer; f += zstride) a.defer[f] = 0;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= TD::Cols) return;
  float part;
  if constexpr (KC == 2) {                                 // two channels per lane
    const int c = 2 * lane;
    float w0 = 0.f, w1 = 0.f;
    if (n < a.nrows) {
      const uint32_t raw = *reinterpret_cast<const uint32_t*>(a.w + (int64_t)n * TD::C + c);
      w0 = bflo(raw); w1 = bfhi(raw);
    }
    *reinterpret_cast<uint32_t*>(a.wf + (int64_t)n * TD::C + c) = pack_bf2(w0 * a.ln_w[c], w1 * a.ln_w[c + 1]);
    part = a.ln_b != nullptr ? a.ln_b[c] * w0 + a.ln_b[c + 1] * w1 : 0.f;
  } else {                                                 // one channel per lane
    const int c = lane;
    const float w0 = n < a.nrows ? bf2f(a.w[(int64_t)n * TD::C + c]) : 0.f;
    a.wf[(int64_t)n * TD::C + c] = f2bf(w0 * a.ln_w[c]);
    part = a.ln_b != nullptr ? a.ln_b[c] * w0 : 0.f;
  }
  const float tot = wave_sum(part);
  if (lane == 0) a.off[n] = tot;
}

// ---------------------------------------------------------------------------------------
// 1. LN + projection
// ---------------------------------------------------------------------------------------
struct TriProjArgs {
  int N, NP, H, transpose;
  float qscale;                       // softmax scale * log2(e)
  const uint16_t* z; const uint8_t* seq;
  const uint16_t* wf; const float* off;   // folded weight [Cols, C] and column offsets
  uint16_t *q, *k, *vt, *bias;
  int items, items_per_wave;          // items = NP * NP / 32 position blocks
};

// Persistent: each workgroup keeps the folded weight in LDS and walks 32-position blocks;
// positions of attention row r are z[r, p] (starting node) or z[p, r] (ending node).
// A block of 32 projection rows is one head of 32 dims (KC = 2) or two heads of 16 (KC = 1,
// rows 16 j .. 16 j + 15 = head 2 nb + j).
template <int KC>
__global__ __launch_bounds__(64 * kPWaves) void tri_proj_kernel(const TriProjArgs a) {
  using TD = TriDims<KC>;
  constexpr int C = TD::C, WP = TD::WP, NC = TD::NC, NB = TD::NB, PB = TD::ProjBlocks;
  __shared__ __attribute__((aligned(16))) uint16_t sW[PB * 32 * WP];
  __shared__ __attribute__((aligned(16))) float sOff[PB * 32];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, li = lane & 31;
  const int N = a.N, NP = a.NP, H = a.H;

  // every load is issued before the first LDS store: one memory latency for the whole staging
  // (a loop of load, wait, store paid it 13 times per workgroup)
  constexpr int kPieces = PB * 32 * (C / 8);                // 16-byte pieces of the staged rows
  constexpr int kStage = (kPieces + 64 * kPWaves - 1) / (64 * kPWaves);
  static_assert(KC != 2 || kPieces % (64 * kPWaves) == 0, "whole staging rounds");
  u32x4 wst[kStage];
#pragma unroll
  for (int j = 0; j < kStage; ++j) {
    const int t = tid + j * 64 * kPWaves, n = t / (C / 8), c8 = (t % (C / 8)) * 8;
    const int src = n < 3 * C ? n : n + C;                  // LDS block 3 NB <- folded bias block 4 NB
    if (kPieces % (64 * kPWaves) == 0 || t < kPieces) wst[j] = ld16(a.wf + (int64_t)src * C + c8);
  }
#pragma unroll
  for (int j = 0; j < kStage; ++j) {
    const int t = tid + j * 64 * kPWaves, n = t / (C / 8), c8 = (t % (C / 8)) * 8;
    if (kPieces % (64 * kPWaves) == 0 || t < kPieces) st16(&sW[n * WP + c8], wst[j]);
  }
  for (int n = tid; n < PB * 32; n += 64 * kPWaves) sOff[n] = a.off[n < 3 * C ? n : n + C];
  __syncthreads();

  const int bpr = NP / 32;                              // position blocks per attention row
  auto block_load = [&](int item, u32x4 (&x)[NC], bool& valid, int& r, int& p, int& sm) {
    r = item / bpr;
    p = (item - r * bpr) * 32 + li;
    const int za = a.transpose ? p : r, zb = a.transpose ? r : p;
    valid = za < N && zb < N;
    // the key's sequence mask, loaded with z (the bias below reads it as a bit of a wave ballot):
    // a byte load there, after the stores, had the compiler drain every store before each use
    sm = a.seq[valid ? zb : 0];
    // positions past N read position 0 instead: no branch around the loads, so that the compiler
    // counts them and the stores after them precisely (the LN of an invalid lane is zeroed)
    const uint16_t* zp = a.z + ((int64_t)(valid ? za : 0) * N + (valid ? zb : 0)) * C + 8 * half;
#pragma unroll
    for (int kk = 0; kk < NC; ++kk) x[kk] = ld16(zp + 16 * kk);
  };
  auto pos_valid = [&](int r, int pe) { return a.transpose ? (pe < N && r < N) : (r < N && pe < N); };

  const int first = (blockIdx.x * kPWaves + wave) * a.items_per_wave;
  const int last = min(first + a.items_per_wave, a.items);
  if (first >= last) return;                            // uniform: no barrier follows
  // z of the next two items is in flight while one computes: per item the loads of item + 2 are
  // issued first, and item + 1 (loaded an item earlier) is normalised at the end, after the
  // stores, so that its wait leaves them in flight.  Two register blocks alternate.
  struct ZBlock { u32x4 x[NC]; bool v; int r, p, sm; };
  ZBlock za_, zb_;
  block_load(first, za_.x, za_.v, za_.r, za_.p, za_.sm);
  if (first + 1 < last) block_load(first + 1, zb_.x, zb_.v, zb_.r, zb_.p, zb_.sm);
  bf16x8 xo[NC];
  bool valid = za_.v;
  int r = za_.r, p = za_.p;                             // this lane's position p (= p0 + li)
  ln_operands<NC>(za_.x, valid, xo);
  // bit j: sequence mask of the key of position p0 + j (lanes j and 32 + j hold the same one)
  uint32_t mbits = (uint32_t)__ballot(za_.sm != 0);
  auto iteration = [&](int item, ZBlock& nxt, ZBlock& fut) __attribute__((always_inline)) {
    // the LDS weights are re-read every item: hoisted out of the loop they would not fit in
    // registers
    asm volatile("" ::: "memory");
    if (item + 2 < last) block_load(item + 2, fut.x, fut.v, fut.r, fut.p, fut.sm);
    const int p0 = p - li;

    // q, k: D^T = W . X^T -> lane = position; registers 8*kk .. 8*kk+7 are the 16 bytes of
    // k-chunk kk (KC = 2) or of head 2 nb + kk (KC = 1) in the Q/K layout
#pragma unroll
    for (int which = 0; which < 2; ++which) {
      uint16_t* dst = which == 0 ? a.q : a.k;
      const float sc = which == 0 ? a.qscale : 1.0f;
#pragma unroll
      for (int hh = 0; hh < NB; ++hh) {
        const int nb = NB * which + hh;
        f32x16 acc;
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
        for (int kk = 0; kk < NC; ++kk)
          acc = mfma32(as_bf16x8(ld16(&sW[(32 * nb + li) * WP + 16 * kk + 8 * half])), xo[kk], acc);
        // KC = 2: k-chunk kk of head hh, 512 elements apart; KC = 1: head 2 hh + kk (NP * 16 apart)
        uint16_t* op = dst + ql_off<KC>(r, KC == 2 ? hh : 2 * hh, H, NP, p, 0, half);
        constexpr int kStep = KC == 2 ? 512 : 0;
        const int64_t step = KC == 2 ? kStep : (int64_t)NP * 16;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const f32x4 o0 = *reinterpret_cast<const f32x4*>(&sOff[32 * nb + 16 * kk + 4 * half]);
          const f32x4 o1 = *reinterpret_cast<const f32x4*>(&sOff[32 * nb + 16 * kk + 8 + 4 * half]);
          uint32_t w[4];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            w[e] = pack_bf2(valid ? (acc[8 * kk + 2 * e] + o0[2 * e]) * sc : 0.f,
                            valid ? (acc[8 * kk + 2 * e + 1] + o0[2 * e + 1]) * sc : 0.f);
            w[2 + e] = pack_bf2(valid ? (acc[8 * kk + 4 + 2 * e] + o1[2 * e]) * sc : 0.f,
                                valid ? (acc[8 * kk + 4 + 2 * e + 1] + o1[2 * e + 1]) * sc : 0.f);
          }
          st16_stream(op + kk * step, u32x4{w[0], w[1], w[2], w[3]});
        }
      }
    }
    // v: D = X . W^T -> lane = projection row li (head hh, dim li for KC = 2; head 2 hh + li / 16,
    // dim li % 16 for KC = 1); registers 8*cc .. 8*cc+7 are keys of 16-key chunk cc of this block
    // in PV slot order for lane half `half`
#pragma unroll
    for (int hh = 0; hh < NB; ++hh) {
      const int nb = 2 * NB + hh;
      f32x16 acc;
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
      for (int kk = 0; kk < NC; ++kk)
        acc = mfma32(xo[kk], as_bf16x8(ld16(&sW[(32 * nb + li) * WP + 16 * kk + 8 * half])), acc);
      const float off = sOff[32 * nb + li];
      const int vh = KC == 2 ? hh : 2 * hh + (li >> 4), vd = KC == 2 ? li : li & 15;
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int t0 = 2 * e, t1 = 2 * e + 1;         // slot t -> key 16cc + 8(t/4) + 4half + t%4
          const int k0 = p0 + 16 * cc + 8 * (t0 >> 2) + 4 * half + (t0 & 3);
          const int k1 = p0 + 16 * cc + 8 * (t1 >> 2) + 4 * half + (t1 & 3);
          w[e] = pack_bf2(pos_valid(r, k0) ? acc[8 * cc + t0] + off : 0.f,
                          pos_valid(r, k1) ? acc[8 * cc + t1] + off : 0.f);
        }
        st16_stream(a.vt + vl_off<KC>(r, vh, H, NP, (p0 >> 4) + cc, half, vd), u32x4{w[0], w[1], w[2], w[3]});
      }
    }
    // bias planes: D = X . Wb^T, lane = head li (< H), 4 consecutive positions
    {
      const int nb = 3 * NB;                            // LDS block of the folded bias rows
      f32x16 acc;
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
      for (int kk = 0; kk < NC; ++kk)
        acc = mfma32(xo[kk], as_bf16x8(ld16(&sW[(32 * nb + li) * WP + 16 * kk + 8 * half])), acc);
      if (li < H) {
        const float off = sOff[32 * nb + li];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int pb = p0 + 8 * c + 4 * half;
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int pe = pb + e;
            const int za = a.transpose ? pe : r, zb = a.transpose ? r : pe;
            float b = (acc[4 * c + e] + off) * SF_LOG2E;
            if (zb >= N) b = -INFINITY;
            else if (za >= N) b = 0.f;
            else if (((mbits >> (pe - p0)) & 1u) == 0) b = SF_MASKED_LOGIT;
            v[e] = b;
          }
          if (!a.transpose) {   // za = r: four consecutive keys of one bias row (stored together)
            *reinterpret_cast<u32x2*>(a.bias + bias_off(li, r, pb, NP)) = u32x2{pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3])};
          } else {              // zb = r: one key of four bias rows
#pragma unroll
            for (int e = 0; e < 4; ++e) a.bias[bias_off(li, pb + e, r, NP)] = f2bf(v[e]);
          }
        }
      }
    }
    if (item + 1 < last) {
      ln_operands<NC>(nxt.x, nxt.v, xo);
      int smn = nxt.sm;
      asm volatile("" : "+v"(smn));                    // the mask test stays here, after the stores
      mbits = (uint32_t)__ballot(smn != 0);
      valid = nxt.v; r = nxt.r; p = nxt.p;
    }
  };
  for (int item = first; item < last; item += 2) {
    iteration(item, zb_, za_);
    if (item + 1 < last) iteration(item + 1, za_, zb_);
  }
}

// ---------------------------------------------------------------------------------------
// 3. gate + output projection + residual over the N*N pair positions (blocks.py:286-291):
//      g = LN(z[p]) . W_g^T   (gamma folded into W_g, beta into its offset)
//      out[p] = z[p] + (o[p] * sigmoid(g)) . W_o^T
//    The gate of pair position (za, zb) is the gate the attention row used there for both the
//    starting and the ending node, so it is recomputed here from z instead of being stored.
//    W_g and W_o are resident in LDS; lane = position.  Within each head, o holds its D dims
//    in the order the attention epilogue produces them (lane half hf, register group c,
//    element e -> dim 8c + 4hf + e); W_o's columns are permuted to match when staged.
// ---------------------------------------------------------------------------------------
struct TriOutArgs {
  int N, NP, transpose;
  const uint16_t* o;                  // o_off blocks
  const uint16_t* wo;                 // [C out, C in]
  const uint16_t* wg;                 // folded gate rows [C, C]
  const float* goff;                  // [C]
  const uint16_t* z;                  // [P, C]
  int add_residual;
  uint16_t* out;
  int items, items_per_wave;          // blocks of 32 queries of one attention row: N * ceil(N / 32)
};

// W_o (its columns permuted to the attention epilogue's dim order) and the folded gate rows into
// LDS rows of pitch WP, by NTHR threads: every load first, then the stores (one memory latency).
template <int NTHR, int KC = 2>
__device__ __forceinline__ void stage_out_weights(uint16_t* sW, uint16_t* sG, float* sGoff, const uint16_t* wo,
                                                  const uint16_t* wg, const float* goff, int tid) {
  constexpr int C = TriDims<KC>::C, WP = TriDims<KC>::WP;
  constexpr int kStage = C * (C / 8) / NTHR;
  static_assert(C * (C / 8) % NTHR == 0, "whole staging rounds");
  u32x2 wlo[kStage], whi[kStage];
  u32x4 gst[kStage];
#pragma unroll
  for (int u = 0; u < kStage; ++u) {
    const int t = tid + u * NTHR, n = t / (C / 8), c8 = (t % (C / 8)) * 8;
    // o feature c8 .. c8+7 = (head, lane half hf, groups 2j and 2j+1): natural dims
    // 16j + 4hf + 0..3 and 16j + 8 + 4hf + 0..3 of the head (KC = 1: j = 0)
    const int hd = KC == 2 ? c8 & ~31 : c8 & ~15;
    const int hf = KC == 2 ? (c8 >> 4) & 1 : (c8 >> 3) & 1, j = KC == 2 ? (c8 >> 3) & 1 : 0;
    const uint16_t* src = wo + (int64_t)n * C + hd + 16 * j + 4 * hf;
    wlo[u] = *reinterpret_cast<const u32x2*>(src);
    whi[u] = *reinterpret_cast<const u32x2*>(src + 8);
    gst[u] = ld16(wg + (int64_t)n * C + c8);
  }
#pragma unroll
  for (int u = 0; u < kStage; ++u) {
    const int t = tid + u * NTHR, n = t / (C / 8), c8 = (t % (C / 8)) * 8;
    st16(&sW[n * WP + c8], u32x4{wlo[u][0], wlo[u][1], whi[u][0], whi[u][1]});
    st16(&sG[n * WP + c8], gst[u]);
  }
  for (int n = tid; n < C; n += NTHR) sGoff[n] = goff[n];
}

// Gate of 32 pair positions (lane = position li, half = channel half): from this lane's z
// channels 16 kk + 8 half + 0..7 (zn) and o pieces (on: feature 16 kk + 8 half + 0..7 of o is,
// for KC = 2, head kk/2, piece (hf = kk%2, k-chunk = half) of the epilogue's order; for KC = 1,
// head kk, piece hf = half) it forms the gated o operands xg of the output projection and, with
// add_residual, the residual pieces zr its accumulator layout needs (output features 8c + 4h + e
// of lane half h sit in z chunk 2nb + c/2 of lane half c%2, elements 4h + e: two permlane32 swaps
// per chunk bring them over).
//   g = LN(z[p]) . W_g^T   (gamma folded into W_g, beta into its offset)
template <int KC = 2>
__device__ __forceinline__ void out_gate(const u32x4 (&on)[TriDims<KC>::NC], const u32x4 (&zn)[TriDims<KC>::NC], bool ok,
                                         bool add_residual, const uint16_t* sG, const float* sGoff, int lane,
                                         bf16x8 (&xg)[TriDims<KC>::NC], uint32_t (&zr)[TriDims<KC>::NC][2][2]) {
  constexpr int NC = TriDims<KC>::NC, NB = TriDims<KC>::NB, WP = TriDims<KC>::WP;
  const int half = lane >> 5, li = lane & 31;
  bf16x8 zo[NC];
  ln_operands<NC>(zn, ok, zo);
  if (add_residual) {   // (add_residual false: the caller supplies the residual another way, or none)
#pragma unroll
    for (int kk = 0; kk < NC; ++kk) {
      const auto s02 = __builtin_amdgcn_permlane32_swap(zn[kk][0], zn[kk][2], false, false);
      const auto s13 = __builtin_amdgcn_permlane32_swap(zn[kk][1], zn[kk][3], false, false);
#pragma unroll
      for (int par = 0; par < 2; ++par) {
        zr[kk][par][0] = s02[par];
        zr[kk][par][1] = s13[par];
      }
    }
  }
  // gate block nb: D^T = W_g . X^T -> lane (position, half hf) holds gate row 8c + 4hf + e of the
  // block in register 4c + e.
  //  KC = 2 (block = head nb): o operand chunk kk = 2nb + j of lane half h needs the gate of
  //    half j, register 8h + t -- one permlane32 swap per register pair gets it.
  //  KC = 1 (block = heads 2nb, 2nb + 1): chunk kk = 2nb + j of lane half h needs dims
  //    8(t/4) + 4h + t%4 of head 2nb + j: rows 16j + ..., register 8j + t of the same lane half.
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    f32x16 acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
    for (int kk = 0; kk < NC; ++kk)
      acc = mfma32(as_bf16x8(ld16(&sG[(32 * nb + li) * WP + 16 * kk + 8 * half])), zo[kk], acc);
    float sg[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) sg[r] = sigmoidf_(acc[r] + sGoff[32 * nb + 8 * (r >> 2) + 4 * half + (r & 3)]);
    if constexpr (KC == 2) {
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(sg[t]), __float_as_uint(sg[t + 8]), false, false);
        // sw[0]: gate for chunk 2nb (j = 0), sw[1]: for chunk 2nb + 1 (j = 1), element t
        sg[t] = __uint_as_float(sw[0]);
        sg[t + 8] = __uint_as_float(sw[1]);
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const u32x4 w = on[2 * nb + j];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bf16x2 v = cvt_bf2(bflo(w[e]) * sg[8 * j + 2 * e], bfhi(w[e]) * sg[8 * j + 2 * e + 1]);
        xg[2 * nb + j][2 * e] = v[0];
        xg[2 * nb + j][2 * e + 1] = v[1];
      }
    }
  }
}

// Output projection + residual of the 32 positions: out[p] = z[p] + (o[p] * g[p]) . W_o^T
// (blocks.py:286-291, :366).  st(nb, c, v) receives output channels 32 nb + 8 c + 4 half .. +3 of
// position li as two bf16 pairs; resid(nb, c) gives the same channels of z.
template <int KC = 2, class Store, class Resid>
__device__ __forceinline__ void out_proj(const bf16x8 (&xg)[TriDims<KC>::NC], bool add_residual, const uint16_t* sW,
                                         int lane, Resid resid, Store st) {
  constexpr int NC = TriDims<KC>::NC, NB = TriDims<KC>::NB, WP = TriDims<KC>::WP;
  const int half = lane >> 5, li = lane & 31;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    f32x16 acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
    for (int kk = 0; kk < NC; ++kk)
      acc = mfma32(as_bf16x8(ld16(&sW[(32 * nb + li) * WP + 16 * kk + 8 * half])), xg[kk], acc);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = acc[4 * c + e];
      if (add_residual) {   // output channels 32 nb + 8 c + 4 half .. +3 of z
        const u32x2 zz = resid(nb, c);
        v[0] += bflo(zz[0]); v[1] += bfhi(zz[0]); v[2] += bflo(zz[1]); v[3] += bfhi(zz[1]);
      }
      st(nb, c, u32x2{pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3])});
    }
  }
}

// o piece of feature chunk kk (16 features) for lane half `half`: head kk/2, piece (hf = kk%2,
// k-chunk = half) for KC = 2; head kk, piece hf = half for KC = 1.
template <int KC>
__device__ __forceinline__ int64_t o_piece_off(int kk, int r, int i, int half, int N, int NP) {
  return KC == 2 ? o_off<2>(kk >> 1, r, i, kk & 1, half, N, NP) : o_off<1>(kk, r, i, half, 0, N, NP);
}

template <int KC>
__global__ __launch_bounds__(64 * kPWaves) void tri_out_kernel(const TriOutArgs a) {
  using TD = TriDims<KC>;
  constexpr int C = TD::C, WP = TD::WP, NC = TD::NC;
  __shared__ __attribute__((aligned(16))) uint16_t sW[C * WP];
  __shared__ __attribute__((aligned(16))) uint16_t sG[C * WP];
  __shared__ __attribute__((aligned(16))) float sGoff[C];
  __shared__ __attribute__((aligned(16))) uint16_t sOut[kPWaves][32 * WP];   // per-wave output rows
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, li = lane & 31;
  uint16_t* const so = sOut[wave];
  stage_out_weights<64 * kPWaves, KC>(sW, sG, sGoff, a.wo, a.wg, a.goff, tid);
  __syncthreads();
  const int first = (blockIdx.x * kPWaves + wave) * a.items_per_wave;
  const int last = min(first + a.items_per_wave, a.items);
  // item = (attention row r, block ib of 32 queries); lane li takes query i = 32 ib + li, at pair
  // position (r, i) (starting node) or (i, r) (ending node)
  const int IB = (a.N + 31) >> 5;
  auto pos = [&](int r, int i) -> int64_t { return a.transpose ? (int64_t)i * a.N + r : (int64_t)r * a.N + i; };
  const int64_t ohs = (int64_t)a.N * (a.NP >> 5) * (512 * KC);   // o elements of one head
  auto load = [&](int item, u32x4 (&xo)[NC], u32x4 (&xz)[NC], int& rn, int& in) {
    rn = item / IB;
    in = (item - rn * IB) * 32 + li;
    // lanes past N read query 0 of the row instead (no masked loads): their LN is zeroed and their
    // outputs are never stored, and the MFMAs keep every position in its own column
    const int i = in < a.N ? in : 0;
    const uint16_t* zp = a.z + pos(rn, i) * C + 8 * half;
    const uint16_t* op = a.o + o_piece_off<KC>(0, rn, i, half, a.N, a.NP);
#pragma unroll
    for (int kk = 0; kk < NC; ++kk) {
      // o_piece_off(kk) = o_piece_off(0) + head * ohs (+ 512 for the second piece of a head, KC = 2)
      xo[kk] = ld16(op + (kk / KC) * ohs + (KC == 2 ? (kk & 1) * 512 : 0));
      xz[kk] = ld16(zp + 16 * kk);
    }
  };
  if (first >= last) return;                            // uniform: no barrier follows
  u32x4 on[NC], zn[NC];
  int r, in;
  load(first, on, zn, r, in);
  bf16x8 xg[NC];
  uint32_t zr[NC][2][2];
  out_gate<KC>(on, zn, in < a.N, a.add_residual, sG, sGoff, lane, xg, zr);
  for (int item = first; item < last; ++item) {
    asm volatile("" ::: "memory");                      // LDS weights are re-read every item
    const int i0 = in - li;
    // the next item's o and z land during this item's projection and stores; its gate is formed
    // at the end of this iteration, after the stores, so the wait for them leaves the stores in
    // flight
    const bool more = item + 1 < last;
    int rn = 0, inn = 0;
    if (more) load(item + 1, on, zn, rn, inn);
    out_proj<KC>(xg, a.add_residual, sW, lane,
                 [&](int nb, int c) { return u32x2{zr[2 * nb + (c >> 1)][c & 1][0], zr[2 * nb + (c >> 1)][c & 1][1]}; },
                 [&](int nb, int c, u32x2 v) { *reinterpret_cast<u32x2*>(so + li * WP + 32 * nb + 4 * half + 8 * c) = v; });
    // the wave's 32 output rows (2 KC KB of contiguous memory for the starting node, 32 rows of
    // 2 C bytes for the ending node): lane (row, 16-byte chunk) stores 16 bytes, 512 / C whole
    // rows per streaming store (the LDS rows were written by other lanes of this wave; LDS
    // executes a wave's accesses in order).  Against 8-byte stores straight from the MFMA layout:
    // 0.128 -> 0.106 ms at N=768, C = 128.
    asm volatile("" ::: "memory");
    constexpr int kRows = 512 / C;                       // rows per store instruction
#pragma unroll
    for (int u = 0; u < 32 / kRows; ++u) {
      // rows past N store the block's last valid row again (identical bytes): no branch
      const int row = min(kRows * u + lane / (C / 8), a.N - 1 - i0), ch = lane % (C / 8);
      const u32x4 v = ld16(so + row * WP + 8 * ch);
      st16_stream(a.out + pos(r, i0 + row) * C + 8 * ch, v);
    }
    if (more) {
      out_gate<KC>(on, zn, inn < a.N, a.add_residual, sG, sGoff, lane, xg, zr);
      r = rn; in = inn;
    }
  }
}

struct TriAttnArgs {
  int N, NP, H, transpose;
  float sum_limit;                    // weight sums outside [2^-100, sum_limit] flag the (row, head)
  const uint16_t *q, *k, *vt, *bias;
  const uint8_t* seq;
  uint16_t* o;                        // o_off blocks: per (head, attention row, 32 queries), N * NP * H * D
  uint8_t* flags;                     // [N][H]: 1 = recomputed exactly (dense: tri_fixup_kernel)
  // block-sparse rows (tri_ibs_tile_attn_kernel): maps [N][H][T][S] of (key block, weight);
  // sparse != 0 also keeps tri_fixup_kernel to the masked rows (flagged rows are recomputed by
  // the exact block-sparse kernel)
  const int32_t* index; const float* weight;
  int T, S, sparse;
  // fused epilogue (tri_attn_fused_kernel / tri_post_kernel): gate, output projection and residual
  const uint16_t* wo;                 // [128 out, 128 in]
  const uint16_t* wg;                 // folded gate rows [128, 128]
  const float* goff;                  // [128]
  const uint16_t* z;                  // [N, N, 128]
  uint16_t* out;                      // [N, N, 128]
  int add_residual;
  int* ctr;                           // [G] heads published per group (1 + XCD id << 8 each), then
                                      // [G] the error word (a wait timed out, or a group spanned XCDs)
  uint8_t* defer;                     // [N] 1: row left to tri_post_kernel (a head of the row was flagged)
  int groups;                         // G
  // row groups to compute (rgl[0] = count, then their indices; null: all NP/4): tasks of row
  // groups whose rows are all masked or past N are not run (the fix-up kernel writes masked rows)
  const int* rgl;
};

constexpr int kTR = 4;                // rows per workgroup
constexpr int kKT = 64;               // keys per tile
constexpr int kAW = 8;                // waves per attention workgroup (256 queries)
constexpr int kPrioUnits = 6;         // units of a tile the younger wave of each SIMD runs at raised priority
// Per-wave table of the block-sparse kernel: the weights of the selected key blocks of its query
// tile for the task's 4 rows, [row][block] floats (0 = not selected), blocks < 128 (N <= 4096).
constexpr int kIbsTabBlocks = 128;
constexpr int kIbsTabBytes = kAW * kTR * kIbsTabBlocks * 4;
// LDS of the fused epilogue: W_o (permuted), W_g (folded), the gate offsets, and the partial sums
// and mean of V of a fully masked row.
constexpr int kFusedW = kPC * kWP * 2;
constexpr int kFusedBytes = 2 * kFusedW + kPC * 4 + 5 * kPC * 4;
// Bound of a fused epilogue wait (iterations of a 64-cycle sleep, ~0.1 s): every wait is for
// work that resident workgroups finish on their own, so only a broken assumption (a workgroup
// that never runs) reaches it; the rows concerned are then written as NaN and the error word set.
constexpr int kFusedSpin = 1 << 20;

typedef __attribute__((address_space(3))) uint32_t lds_u32;

// One LDS tile buffer, all in 16-byte slots; every 1 KB of it is filled by one
// global_load_lds_dwordx4 (lane L -> bytes 16L..16L+15):
//   K    [row rr][key block 2][k-chunk KC][lane half 2][key 32]   copied as stored     8 KC KB
//   V^T  [row rr][16-key chunk 4][lane half 2][dim 16 KC]        copied as stored     8 KC KB
// The operand reads of consecutive lanes are consecutive slots (bank-conflict free), and
// every read of a lane is one per-lane base plus a compile-time offset.  The bias tile is not
// staged here: each wave's 32 query rows of it are its own (no other wave reads them), so every
// wave loads them a tile ahead straight into registers, which takes them off the LDS (a DMA
// write and a read per byte) and out of the barrier's wait.
template <int KC>
struct TileLayout {
  static constexpr int kRowBytes = kKT * 16 * KC * 2;       // K (or V^T) of one row
  static constexpr int kKBytes = kTR * kRowBytes;
  static constexpr int kVBytes = kTR * kRowBytes;
  static constexpr int kKVBytes = kKBytes + kVBytes;
  static constexpr int kBytes = kKVBytes;
  __device__ static constexpr int chunk_offset(int buf, int c) { return buf * kKVBytes + c * 1024; }
  static constexpr int kChunks = kBytes / 1024;
  static constexpr int kChunksPerWave = kChunks / kAW;
  static_assert(kChunks % kAW == 0, "tile chunks must split evenly over the waves");
  static_assert(kChunksPerWave == 2 * KC && kAW == 2 * kTR,
                "waves 0-3 copy K rows, waves 4-7 V^T rows, 2 KC chunks each");
};

// Task = (head, row group of 4 rows, block of 256 queries).  The grid is persistent: at most
// one workgroup per CU (its 8 waves use 2 waves' worth of registers on every SIMD), each walking
// its tasks with the tile pipeline running straight through task boundaries -- the last tile of a
// task loads the first tile of the next one, and the next task's Q operands are loaded while the
// last tile computes.  With one short-lived workgroup per task the prologue (Q and first-tile
// loads, nothing to overlap them with) and the epilogue cost 23% of the kernel.
// Workgroup b is assumed to run on XCD b % 8 (round-robin dispatch) and takes the tasks
// x * T/8 + b/8 + (G/8) j of XCD x's contiguous range, so the workgroups an XCD runs together
// share one head's bias plane and neighbouring row groups' K/V tiles in its L2.
//
// SP (tri_ibs_tile_attn_kernel): block-sparse rows on the same pipeline.  At the start of a task
// each wave fills its table from the maps; a unit (row rr, 32-key block b) whose weight w is 0 is
// skipped (no S^T MFMAs, exponentials or P.V), and a selected one adds log2 w to its logits, so
// that its weights are w 2^s.  Row sums, normalisation and the out-of-range flags are unchanged.
template <bool SP, bool FUSED, int KC = 2>
__device__ __forceinline__ void tri_attn_body(const TriAttnArgs& a) {
  static_assert(!(SP && FUSED), "the block-sparse rows use the separate output stage");
  static_assert(KC == 2 || (!SP && !FUSED), "head dim 16: dense rows, separate output stage");
  using TL = TileLayout<KC>;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * TL::kBytes + (SP ? kIbsTabBytes : 0) + (FUSED ? kFusedBytes : 0)];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: scalar branches
  const int half = lane >> 5, li = lane & 31;
  const int N = a.N, NP = a.NP, H = a.H;

  const int QB = (NP + 32 * kAW - 1) / (32 * kAW), RG = NP / kTR;
  // row groups to run: the list of those with a valid row, or all (FUSED: the epilogue writes
  // every row, masked ones included)
  const int nrg = (!FUSED && a.rgl != nullptr) ? __builtin_amdgcn_readfirstlane(a.rgl[0]) : RG;
  const int total = QB * nrg * H;
  const int per = (total + 7) / 8;                  // tasks per XCD (FUSED: exact, a multiple of 4)
  const int xcd = blockIdx.x & 7, G8 = gridDim.x >> 3;
  const int xper = max(0, min(per, total - xcd * per));   // this XCD's tasks (the last may have fewer)
  int task = blockIdx.x >> 3;                       // index within the XCD's range
  if (task >= xper) return;                         // uniform over the workgroup
  // FUSED: the heads are innermost, so that the 4 tasks of a group (row group, query block) are
  // tasks 4m .. 4m+3 of an XCD's range, run in the same round by workgroups 4m' .. 4m'+3 of that
  // XCD (G8 is a multiple of 4): one L2 holds the o of all 4 heads for the group's epilogue.
  // (Measured on the attention alone: +3%, the bias planes of all heads then share the L2.)
  auto decode = [&](int tl, int& r0, int& h, int& qb) __attribute__((always_inline)) {
    const int t = xcd * per + tl;
    if constexpr (FUSED) {
      h = t & 3;
      qb = (t >> 2) % QB;
      r0 = ((t >> 2) / QB) * kTR;
    } else {
      qb = t % QB;
      const int k = (t / QB) % nrg;
      r0 = ((!FUSED && a.rgl != nullptr) ? __builtin_amdgcn_readfirstlane(a.rgl[1 + k]) : k) * kTR;
      h = t / (QB * nrg);
    }
  };

  // ---- tile loader: this wave's 1 KB chunks of a tile, straight into LDS.  Wave w < 4 copies
  //      the K tile of row r0 + w, wave w >= 4 the V^T tile of row r0 + w - 4: four 1 KB quarters
  //      of 4 KB of contiguous memory. ----
  const int64_t rstride = (int64_t)H * NP * 16 * KC;        // row stride of the Q/K/G and V^T layouts
  const uint32_t lane16 = (uint32_t)lane * 16u;
  auto loader_src = [&](int r0, int h) __attribute__((always_inline)) -> const char* {
    return wave < 4 ? (const char*)(a.k + ql_off<KC>(r0 + wave, h, H, NP, 0, 0, 0))
                    : (const char*)(a.vt + vl_off<KC>(r0 + wave - 4, h, H, NP, 0, 0, 0));
  };
  auto load_tile = [&](const char* wsrc, int j0, int buf) __attribute__((always_inline)) {
    const char* src = wsrc + (int64_t)j0 * (32 * KC);        // K / V^T bytes per key
#pragma unroll
    for (int u = 0; u < TL::kChunksPerWave; ++u)
      __builtin_amdgcn_global_load_lds(src + u * 1024 + lane16,
                                       (lds_u32*)(smem + TL::chunk_offset(buf, wave * TL::kChunksPerWave + u)), 16, 0, 0);
  };
  auto kslot = [&](int buf, int rr, int kb, int kk) __attribute__((always_inline)) -> const uint8_t* {
    return smem + buf * TL::kKVBytes + rr * TL::kRowBytes + (kb * 2 * KC + kk * 2 + half) * 512 + li * 16;
  };
  // V^T rows of the P.V MFMA's A operand: dims 0 .. 16 KC - 1 (KC = 1: lanes li >= 16 read dims
  // li - 16 again; output rows 16..31 of that MFMA are not used)
  auto vslot = [&](int buf, int rr, int c16) __attribute__((always_inline)) -> const uint8_t* {
    return smem + buf * TL::kKVBytes + TL::kKBytes + rr * TL::kRowBytes + (c16 * 2 + half) * (256 * KC)
           + (KC == 2 ? li : li & 15) * 16;
  };
  // ---- this lane's bias of a tile, straight into registers: piece k of the wave's 4 KB block
  //      (bias_off_stored) is pieces 4(k/2) + 2 half + k%2 of its query's 64 keys, 8 keys each:
  //      the keys its S^T registers hold.  Query tiles past the last are clamped (idle waves). ----
  u32x4 breg[4];
  auto bias_src = [&](int h, int qb) __attribute__((always_inline)) -> const char* {
    const int qt = min(qb * kAW + wave, (NP >> 5) - 1);
    return (const char*)(a.bias + (((int64_t)h * (NP >> 5) + qt) * (NP >> 6) << 11)) + lane16;
  };
  auto load_bias_regs = [&](const char* bsrc, int j0) __attribute__((always_inline)) {
    const char* p = bsrc + (int64_t)j0 * 64;             // 4 KB per 64-key tile
#pragma unroll
    for (int k = 0; k < 4; ++k) breg[k] = ld16(p + 1024 * k);
  };

  // Q operands (B of S^T = K Q^T) of a task's 4 rows.  Rows past N hold zeros and are never stored.
  bf16x8 qb8[kTR][KC];
  auto load_q = [&](int r0, int h, int qb, bf16x8 (&qd)[kTR][KC]) __attribute__((always_inline)) {
    const int iq = min(qb * 32 * kAW + 32 * wave + li, NP - 1);   // operand row (results of i >= N unused)
    const uint16_t* qbase = a.q + ql_off<KC>(r0, h, H, NP, iq, 0, half);
#pragma unroll
    for (int rr = 0; rr < kTR; ++rr)
#pragma unroll
      for (int kk = 0; kk < KC; ++kk) qd[rr][kk] = as_bf16x8(ld16(qbase + rr * rstride + kk * 512));
  };
  // Softmax against a fixed reference point of 0: the logits (log2 units, q carries
  // scale * log2 e) are exponentiated as they come out of the S^T MFMA, with no running maximum
  // and no rescaling of o.  Logits of realistic inputs lie far inside the range where that is
  // exact in fp32/bf16 (2^+-100); a row whose weight sum leaves [2^-100, sum_limit] -- an
  // overflow, an underflow of the whole row, or a forced test limit -- is flagged at the end
  // and recomputed with an exact two-pass softmax by tri_fixup_kernel.  A weight w <= sum <=
  // 2^100 cannot overflow, and o = sum_k w_k v_k stays finite for any bf16 v of moderate size.
  f32x16 o[kTR];
  f32x4 lsum[kTR];
  // Row sums on the matrix core: a 16x16x32 MFMA whose B operand is the P^T chunk of the P.V
  // MFMA (lane l: query l%32, keys of lane group l/16) and whose A operand selects lane groups
  // {0, 2} into output rows 0..7 and {1, 3} into rows 8..15.  Output (m, n) is then the sum over
  // the chunk's 16 keys of query n (m < 8) or query n + 16 (m >= 8).
  bf16x8 sel;
#pragma unroll
  for (int e = 0; e < 8; ++e) sel[e] = (__bf16)((((lane & 15) < 8) == (((lane >> 4) & 1) == 0)) ? 1.0f : 0.0f);

  // bias tile of this wave's 32 queries (in breg) -> fp32 accumulator seed in S^T register order
  f32x16 bseed[2];
  auto load_bias = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const u32x4 b0 = breg[2 * kb];
      const u32x4 b1 = breg[2 * kb + 1];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        bseed[kb][2 * e] = bflo(b0[e]);
        bseed[kb][2 * e + 1] = bfhi(b0[e]);
        bseed[kb][8 + 2 * e] = bflo(b1[e]);
        bseed[kb][8 + 2 * e + 1] = bfhi(b1[e]);
      }
    }
  };
  auto load_k = [&](int rr, int kb, int buf, bf16x8 (&kr)[KC]) __attribute__((always_inline)) {
#pragma unroll
    for (int kk = 0; kk < KC; ++kk) kr[kk] = as_bf16x8(ld16(kslot(buf, rr, kb, kk)));
  };
  auto load_v = [&](int rr, int kb, int buf, bf16x8 (&vr)[2]) __attribute__((always_inline)) {
    vr[0] = as_bf16x8(ld16(vslot(buf, rr, 2 * kb)));
    vr[1] = as_bf16x8(ld16(vslot(buf, rr, 2 * kb + 1)));
  };
  // S^T half of unit (row rr, 32-key half kb) = K Q^T + bias, logits in log2 units
  auto qk = [&](int rr, int kb, const bf16x8 (&kr)[KC], f32x16& s) __attribute__((always_inline)) {
    if constexpr (KC == 2) s = mfma32(kr[1], qb8[rr][1], mfma32(kr[0], qb8[rr][0], bseed[kb]));
    else s = mfma32(kr[0], qb8[rr][0], bseed[kb]);
  };

  // The work of a tile is split into units (row rr, 32-key half kb): S^T half = 32 keys x 32
  // queries (2 MFMAs), its 16 weights per lane, their P.V (2 MFMAs) and row sums (2 small
  // MFMAs).  Units are software-pipelined: the S^T MFMAs of unit u+1 are issued before the
  // exponentials of unit u, K operands are read two units ahead and V operands one unit ahead.
  // The scheduling fences keep the compiler from sinking those reads to their uses (which
  // exposed the LDS latency every unit) and from hoisting unit u+1's S^T MFMAs away from the
  // exponentials they overlap.
  // RELOAD (the last tile of a task): row rr's Q operands are replaced by the next task's (nq:
  // this lane's Q of that task) as soon as the S^T MFMA of unit 2rr+1 -- their last use -- has
  // been issued, so that those loads have most of a tile to land.
  // SP: wu[u] = weight of unit u of the current tile (wave-uniform scalars), 0 = skipped
  float wu[2 * kTR];
  auto on = [&](int u) __attribute__((always_inline)) { return !SP || wu[u] != 0.f; };
  // ISSUE(u), u < 4: the next tile's loads, one K/V^T chunk (units u < 2 KC) and one bias piece
  // per unit (see the tile below).  PRIO: the wave's raised issue priority is dropped at unit
  // kPrioUnits.
  // FIN(rr): row rr's result is final (its last P.V MFMA was issued a unit earlier): the last tile
  // of a task normalises and stores rows 0..2 there, spread over the tile, instead of all four
  // rows of all eight waves storing together after it.
  auto units = [&](int buf, auto reloadc, const uint16_t* nq, auto issue, auto fin) __attribute__((always_inline)) {
    constexpr bool RELOAD = decltype(reloadc)::value;
    f32x16 sc, sn;
    bf16x8 kr[KC], vr[2];
    if (on(0)) {
      load_k(0, 0, buf, kr);
      qk(0, 0, kr, sc);
    }
    if (on(1)) load_k(0, 1, buf, kr);
    if (on(0)) load_v(0, 0, buf, vr);
#pragma unroll
    for (int u = 0; u < 2 * kTR; ++u) {
      const int rr = u >> 1;
      if (u < 4) {
        issue(u);
        asm volatile("" ::: "memory");   // keeps the loads in issue order (the tile's waits count them)
      }
      if (u == kPrioUnits && wave >= 4) __builtin_amdgcn_s_setprio(0);
      if (u + 1 < 2 * kTR && on(u + 1)) qk((u + 1) >> 1, (u + 1) & 1, kr, sn);
      if (u + 2 < 2 * kTR && on(u + 2)) load_k((u + 2) >> 1, (u + 2) & 1, buf, kr);
      if (RELOAD && (u & 1) == 0) {
#pragma unroll
        for (int kk = 0; kk < KC; ++kk) qb8[rr][kk] = as_bf16x8(ld16(nq + rr * rstride + kk * 512));
      }
      __builtin_amdgcn_sched_barrier(0);
      if (on(u)) {
        if (SP && wu[u] != 1.0f) {     // a drawn block: weights w 2^s = 2^(s + log2 w)
          const float lw = __builtin_amdgcn_logf(wu[u]);
#pragma unroll
          for (int e = 0; e < 16; ++e) sc[e] += lw;
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          bf16x8 pb;                     // P^T chunk 2kb+j: weights 2^s as bf16 pairs
#pragma unroll
          for (int q2 = 0; q2 < 4; ++q2) {
            const bf16x2 w = cvt_bf2(fast_exp2(sc[8 * j + 2 * q2]), fast_exp2(sc[8 * j + 2 * q2 + 1]));
            pb[2 * q2] = w[0];
            pb[2 * q2 + 1] = w[1];
          }
          o[rr] = mfma32(vr[j], pb, o[rr]);
          lsum[rr] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sel, pb, lsum[rr], 0, 0, 0);
        }
      }
      if (u + 1 < 2 * kTR && on(u + 1)) load_v((u + 1) >> 1, (u + 1) & 1, buf, vr);
      __builtin_amdgcn_sched_barrier(0);
      sc = sn;
      if ((u & 1) == 0 && u >= 2) fin((u >> 1) - 1);
    }
  };
  // SP: this wave's table (weights of its query tile's selected blocks for the task's 4 rows)
  float* tab = reinterpret_cast<float*>(smem + 2 * TL::kBytes) + wave * kTR * kIbsTabBlocks;
  auto fill_table = [&](int r0, int h, int qb) __attribute__((always_inline)) {
    asm volatile("" ::: "memory");
    for (int e = lane; e < kTR * kIbsTabBlocks; e += 64) tab[e] = 0.f;
    const int t = qb * kAW + wave;                           // this wave's query tile
    const int ne = kTR * a.S;                                // <= 256 entries: 4 per lane
    int bs[4];
    float ws[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int e = lane + 64 * k, rr = e / a.S, r = r0 + rr;
      bs[k] = -1;
      ws[k] = 0.f;
      if (e < ne && t < a.T && r < N) {
        const int64_t m = (((int64_t)r * H + h) * a.T + t) * a.S + (e - rr * a.S);
        bs[k] = a.index[m];
        ws[k] = a.weight[m];
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int rr = (lane + 64 * k) / a.S;
      // unused slot: index out of range or weight <= 0 (the exact kernel skips the same)
      if (bs[k] >= 0 && bs[k] < a.T && ws[k] > 0.f) atomicAdd(&tab[rr * kIbsTabBlocks + bs[k]], ws[k]);
    }
    asm volatile("" ::: "memory");
  };
  auto tile_weights = [&](int tt) __attribute__((always_inline)) {
#pragma unroll
    for (int rr = 0; rr < kTR; ++rr) {
      const f32x2 v = *reinterpret_cast<const f32x2*>(tab + rr * kIbsTabBlocks + 2 * tt);
      wu[2 * rr] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v[0])));
      wu[2 * rr + 1] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v[1])));
    }
  };

  const int ntiles = NP / kKT;
  const int q32 = lane & 31;
  const int src_lane = q32 < 16 ? q32 : q32 + 16;   // a lane whose row-sum output holds query q32

  // ---- FUSED: the gate, output projection and residual of a group's rows, in the epilogue ----
  // A task publishes its group (row group, query block) once its o stores are in L2: the group's
  // count grows by 1 + (XCD id << 8).  One task later -- when the group's other three heads,
  // started in the same round, are done as well -- the workgroup that ran head h writes the
  // output of the group's row r0 + h (256 queries, one 32-query item per wave): o of the four
  // heads from this XCD's L2, z for the gate and the residual, out = z + (o * g) W_o.
  uint16_t* const sWo = reinterpret_cast<uint16_t*>(smem + 2 * TL::kBytes);
  uint16_t* const sWg = sWo + kPC * kWP;
  float* const sGoff = reinterpret_cast<float*>(sWg + kPC * kWP);
  float* const sPart = sGoff + kPC;                          // [4][128] partial sums of V
  float* const sMean = sPart + 4 * kPC;                      // [128] mean of V (head-major)
  const int xcc = FUSED ? (int)__builtin_amdgcn_s_getreg((3 << 11) | 20) : 0;   // HW_REG_XCC_ID[3:0]
  auto pos_of = [&](int r, int i) __attribute__((always_inline)) -> int64_t {
    return a.transpose ? (int64_t)i * N + r : (int64_t)r * N + i;
  };
  auto publish = [&](int gid) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0);                           // this wave's o stores and flags are in L2
    __syncthreads();                                         // ... and every other wave's
    if (tid == 0) __hip_atomic_fetch_add(a.ctr + gid, 1 + (xcc << 8), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  auto outwork = [&](int gid, int r, int oqb) __attribute__((always_inline)) {
    int v = 0;
    for (int it = 0; it < kFusedSpin; ++it) {                // uniform: every lane reads the same word
      v = __builtin_amdgcn_readfirstlane(__hip_atomic_load(a.ctr + gid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      if ((v & 0xff) >= 4) break;
      __builtin_amdgcn_s_sleep(1);
    }
    if (r >= N) return;                                      // a padding row of the group
    const int i0 = (oqb * kAW + wave) * 32, i = i0 + li;
    const bool ok = i < N;
    auto store = [&](int nb, int c, u32x2 val) __attribute__((always_inline)) {
      if (ok) *reinterpret_cast<u32x2*>(a.out + pos_of(r, i) * kPC + 32 * nb + 8 * c + 4 * half) = val;
    };
    if (v != 4 + ((4 * xcc) << 8)) {
      // the wait timed out, or the group's heads ran on different XCDs (no common L2): the rows
      // are written as NaN and the error word is set, never a stale or partial result
      if (tid == 0) a.ctr[a.groups] = 1;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int c = 0; c < 4; ++c) store(nb, c, u32x2{0x7fc07fc0u, 0x7fc07fc0u});
      return;
    }
    // a flagged head: tri_post_kernel recomputes the row exactly and writes its output (all of
    // its query blocks: each of the row's groups marks it, the mark is idempotent)
    const uint32_t fl = __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(reinterpret_cast<uint32_t*>(a.flags + r * 4), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    if (fl != 0) {
      if (tid == 0) a.defer[r] = 1;
      return;
    }
    u32x4 on[8];
    if (a.seq[r] == 0) {
      // every logit of a masked row is the masked value, so the reference's softmax is uniform:
      // o = mean of V over all N keys (keys past N hold V = 0); thread (part, head, dim)
      {
        const int hd = tid & 127, hh = hd >> 5, d = hd & 31, pp = tid >> 7;
        const int per_part = NP / 64;                        // 16-key chunks per part, even
        float s0 = 0.f, s1 = 0.f;
        for (int c16 = pp * per_part; c16 < (pp + 1) * per_part; c16 += 2) {
          u32x4 vv[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) vv[u] = ld16(a.vt + vl_off(r, hh, H, NP, c16 + (u >> 1), u & 1, d));
#pragma unroll
          for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) { s0 += bflo(vv[u][e]); s1 += bfhi(vv[u][e]); }
        }
        sPart[pp * kPC + hd] = s0 + s1;
      }
      __syncthreads();
      if (tid < kPC) sMean[tid] = (sPart[tid] + sPart[kPC + tid] + sPart[2 * kPC + tid] + sPart[3 * kPC + tid]) / (float)N;
      __syncthreads();
      // piece (hf = kk%2, k-chunk = half) of head kk/2: dims 16 half + 8 (t/4) + 4 hf + t%4
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const float* mh = sMean + 32 * (kk >> 1) + 16 * half + 4 * (kk & 1);
        on[kk] = u32x4{pack_bf2(mh[0], mh[1]), pack_bf2(mh[2], mh[3]), pack_bf2(mh[8], mh[9]), pack_bf2(mh[10], mh[11])};
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < 8; ++kk)
        on[kk] = ok ? ld16(a.o + o_off(kk >> 1, r, i, kk & 1, half, N, NP)) : u32x4{0, 0, 0, 0};
    }
    if (i0 < N) {
      u32x4 zn[8];
      const uint16_t* zp = a.z + pos_of(r, ok ? i : 0) * kPC + 8 * half;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) zn[kk] = ok ? ld16(zp + 16 * kk) : u32x4{0, 0, 0, 0};
      // The weights lie above the first 64 KB of LDS, past a ds_read's immediate offset: left
      // alone, the compiler hoisted one base register per weight row block out of the persistent
      // loop and spilled.  An opaque zero makes the bases local to this item.
      int lz = 0;
      asm volatile("" : "+v"(lz));
      const uint16_t* wg_l = sWg + lz;
      const uint16_t* wo_l = sWo + lz;
      bf16x8 xg[8];
      uint32_t zr[8][2][2];                                  // unused: the residual is re-read below
      out_gate(on, zn, ok, false, wg_l, sGoff, lane, xg, zr);
      // the residual straight from z in the accumulator layout (the lines were just read)
      const uint16_t* zq = a.z + pos_of(r, ok ? i : 0) * kPC + 4 * half;
      out_proj(xg, a.add_residual, wo_l, lane,
               [&](int nb, int c) { return ok ? *reinterpret_cast<const u32x2*>(zq + 32 * nb + 8 * c) : u32x2{0, 0}; },
               store);
    }
  };

  int r0, h, qb;
  decode(task, r0, h, qb);
  const char* wsrc = loader_src(r0, h);
  const char* bsrc = bias_src(h, qb);
  load_tile(wsrc, 0, 0);
  load_bias_regs(bsrc, 0);
  if constexpr (FUSED) stage_out_weights<64 * kAW>(sWo, sWg, sGoff, a.wo, a.wg, a.goff, tid);
  __builtin_amdgcn_s_waitcnt(0);                           // this wave's chunks have landed
  __syncthreads();                                         // ... and everybody else's
  load_q(r0, h, qb, qb8);
  bool qready = true;                                      // qb8 holds this task's Q operands (uniform)
  int prev_gid = -1, prev_row = 0, prev_qb = 0;            // FUSED: the previous task's group
  for (;;) {
    const int next = task + G8;
    const bool has_next = next < xper;                     // uniform
    int nr0 = 0, nh = 0, nqb = 0;
    const char* nsrc = wsrc;
    const char* nbsrc = bsrc;
    if (has_next) {
      decode(next, nr0, nh, nqb);
      nsrc = loader_src(nr0, nh);
      nbsrc = bias_src(nh, nqb);
    }
    const int i = qb * 32 * kAW + 32 * wave + li;          // this lane's query
    const bool active = qb * 32 * kAW + 32 * wave < NP;    // uniform: the wave has queries below NP
    // normalise row rr of the task and store it at the pair position (the gate is applied by the
    // output kernel, which recomputes it from z)
    auto finish_row = [&](int rr) __attribute__((always_inline)) {
      if (i >= N) return;
      const int r = r0 + rr;
      const float lt = __shfl(lsum[rr][0], src_lane);
      if (r >= N) return;
      if (!(lt >= 0x1p-100f && lt <= a.sum_limit) && a.seq[r] != 0) a.flags[r * H + h] = 1;
      const float inv = fast_rcp(lt);
#pragma unroll
      for (int kk = 0; kk < KC; ++kk) {                    // O^T rows 16 kk .. 16 kk + 15 (dims)
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          w[e] = pack_bf2(o[rr][8 * kk + 2 * e] * inv, o[rr][8 * kk + 2 * e + 1] * inv);
        // FUSED: plain stores, so that the group's epilogue finds them in L2
        if constexpr (FUSED) st16(a.o + o_off<KC>(h, r, i, half, kk, N, NP), u32x4{w[0], w[1], w[2], w[3]});
        else st16_stream(a.o + o_off<KC>(h, r, i, half, kk, N, NP), u32x4{w[0], w[1], w[2], w[3]});
      }
    };
    if constexpr (SP) fill_table(r0, h, qb);
#pragma unroll
    for (int rr = 0; rr < kTR; ++rr) {
#pragma unroll
      for (int e = 0; e < 16; ++e) o[rr][e] = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) lsum[rr][e] = 0.f;
    }
    // One tile: its bias registers are turned into the S^T seed, then the loads of the tile after
    // it (or of the next task's first tile) are issued -- K/V^T chunks into the other LDS buffer,
    // then the bias into the registers just freed -- and land while it computes.  At its end
    // every wave waits for its chunks and the barrier makes everybody's visible; the bias loads,
    // the youngest, stay in flight.  The first and last tiles of a task are separate code
    // instances: the last one loads the next task's Q operands (into the registers of rows it has
    // finished with), the first one waits for them -- with a wait the compiler sees, so that it
    // puts no conservative wait of its own in front of the first S^T MFMA, where it would also
    // wait for the tile loads just issued.  A plain __syncthreads would also wait for the Q loads
    // at the end of the last tile.
    // this lane's Q operands of the next task (of this task again on the last one: a harmless reload)
    const uint16_t* nq = has_next ? a.q + ql_off<KC>(nr0, nh, H, NP, min(nqb * 32 * kAW + 32 * wave + li, NP - 1), 0, half)
                                  : a.q + ql_off<KC>(r0, h, H, NP, min(qb * 32 * kAW + 32 * wave + li, NP - 1), 0, half);
    auto tile = [&](int tt, auto firstc, auto lastc, auto bufc) __attribute__((always_inline)) {
      constexpr bool FIRST = decltype(firstc)::value, LAST = decltype(lastc)::value;
      constexpr int buf = decltype(bufc)::value;             // compile-time: the compiler then
                                                             // sees that no LDS read of this tile
                                                             // aliases the loads into the other
      if (FIRST) {
        if (!qready) load_q(r0, h, qb, qb8);
        __builtin_amdgcn_s_waitcnt(0x0F70);                  // vmcnt(0): this task's Q operands and bias
      }
      if (active) {                                          // (idle waves need no Q operands or bias)
        if constexpr (SP) {
          tile_weights(tt);
          bool any = false;
#pragma unroll
          for (int u = 0; u < 2 * kTR; ++u) any |= wu[u] != 0.f;
          if (any) load_bias();
        } else {
          load_bias();
        }
      }
      // the seed is read out of breg before the loads below overwrite it
      __builtin_amdgcn_sched_barrier(0);
      // the tile after this one; after the last tile, the next task's first tile (the last task
      // loads its own first tile again: unused, but the code stays branch-free).  A wave issues
      // them one K/V^T chunk and one bias piece per unit over the first 4 units: all 64 issued at
      // the tile start, the later ones waited for room in the CU's memory-instruction queue,
      // holding their waves for ~1000 cycles per tile.
      const char* tsrc = LAST ? nsrc : wsrc;
      const char* tbsrc = LAST ? nbsrc : bsrc;
      const int tj = LAST ? 0 : (tt + 1) * kKT;
      constexpr int kKeyBytes = 32 * KC;                     // K / V^T bytes per key
      // The end-of-tile waits below (KC = 2: `vmcnt(1)` / `vmcnt(5)`) are counts of this lambda's
      // loads in the order they are issued: chunk D_u (u < 2 KC), then bias piece B_u, for
      // u = 0..3 (plus the last tile's Q reloads).  The vector memory counter retires loads in issue order, so the wait
      // covers every K/V^T chunk only if no chunk is issued after a load the wait leaves in
      // flight.  The compiler fence between D_u and B_u (and the one after each issue(u) in the
      // unit loop) is what fixes that order; without it the compiler may reorder the two loads
      // and the last chunk can still be in flight when the barrier releases the other waves.
      auto issue = [&](int u) __attribute__((always_inline)) {
        if (u < TL::kChunksPerWave)
          __builtin_amdgcn_global_load_lds(tsrc + (int64_t)tj * kKeyBytes + u * 1024 + lane16,
                                           (lds_u32*)(smem + TL::chunk_offset(buf ^ 1, wave * TL::kChunksPerWave + u)), 16, 0, 0);
        asm volatile("" ::: "memory");   // the chunk before the bias piece (left alone, the compiler
                                         // put the bias load first, and the partial waits below
                                         // then let the last chunk stay in flight past the barrier)
        breg[u] = ld16(tbsrc + (int64_t)tj * 64 + 1024 * u);
      };
      // An idle wave loads its bias pieces as well: on a task's last tile they are the next
      // task's first-tile bias, which the wave needs if it is active there (a workgroup's tasks
      // step through the query blocks when QB does not divide the task stride).
      if (!active) {
        load_tile(tsrc, tj, buf ^ 1);
        load_bias_regs(tbsrc, tj);
      }
      // On each SIMD the wave launched first (w < 4) has the older age, so it won every issue
      // slot it competed for, finished its units ~25% sooner and then waited at the barrier
      // while the younger one (w + 4) ran alone (19% of the kernel at the barrier).  The younger
      // wave gets the higher priority for the first kPrioUnits units of a tile instead.
      if (wave >= 4) __builtin_amdgcn_s_setprio(1);
      // the loads of the tile must stay in issue order with the Q reloads (the partial waits at
      // the end of the tile count on it): no memory operation crosses this point
      asm volatile("" ::: "memory");
      // rows 0..2 of the last tile are finished inside its units (the stores join the loads in the
      // memory counter; the partial waits below still cover the K/V^T chunks, since the loads
      // return in issue order and the stores only add to the count)
      auto fin = [&](int rr) __attribute__((always_inline)) {
        if constexpr (LAST && !SP) finish_row(rr);
      };
      if (active) units(buf, lastc, nq, issue, fin);
      __builtin_amdgcn_s_setprio(0);
      // this wave's chunks landed.  Issue order (unit: loads), KC = 2: 0: D0 B0 [Q0 Q0], 1: D1 B1,
      // 2: D2 B2 [Q1 Q1], 3: D3 B3, 4: [Q2 Q2], 6: [Q3 Q3] -- D chunk, B bias piece, [Q] the last
      // tile's reloads of the next task's Q operands -- so the bias piece of unit 3 and the Q
      // reloads after it may stay in flight (idle waves issued no bias or Q loads: they wait for
      // all).  KC = 1: 0: D0 B0 [Q0], 1: D1 B1, 2: B2 [Q1], 3: B3, 4: [Q2], 6: [Q3] -- the bias
      // pieces of units 1-3 and the Q reloads after D1 may stay in flight.
      static_assert(2 * kTR == 8 && TL::kChunksPerWave == 2 * KC && kPrioUnits >= 0,
                    "the partial waits below count the loads of the unit schedule above");
      if constexpr (KC == 2) {
        if (LAST && active) asm volatile("s_waitcnt vmcnt(5) lgkmcnt(0)" ::: "memory");
        else if (active) asm volatile("s_waitcnt vmcnt(1) lgkmcnt(0)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
      } else {
        if (LAST && active) asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)" ::: "memory");
        else if (active) asm volatile("s_waitcnt vmcnt(3) lgkmcnt(0)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
      }
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    };
    // ntiles is even: every task starts in buffer 0 and ends in buffer 1
    using F = std::false_type; using T = std::true_type;
    using B0 = std::integral_constant<int, 0>; using B1 = std::integral_constant<int, 1>;
    tile(0, T{}, F{}, B0{});
    for (int tt = 1; tt + 1 < ntiles; tt += 2) {
      tile(tt, F{}, F{}, B1{});
      tile(tt + 1, F{}, F{}, B0{});
    }
    tile(ntiles - 1, F{}, T{}, B1{});
    qready = active;                 // an idle wave loaded no Q operands for the next task

    // ---- epilogue: the rows the last tile did not finish (idle waves have no queries below N) ----
#pragma unroll
    for (int rr = SP ? 0 : kTR - 1; rr < kTR; ++rr) finish_row(rr);
    if constexpr (FUSED) {
      // publish this task's group, then write the output row of the previous task's group (its
      // other heads ran in the previous round: no wait in practice); the next task's first
      // tile and Q operands are loading meanwhile
      const int gid = (xcd * per + task) >> 2;
      publish(gid);
      if (prev_gid >= 0) outwork(prev_gid, prev_row, prev_qb);
      prev_gid = gid; prev_row = r0 + h; prev_qb = qb;
    }
    if (!has_next) break;
    task = next; r0 = nr0; h = nh; qb = nqb; wsrc = nsrc; bsrc = nbsrc;
  }
  if constexpr (FUSED) outwork(prev_gid, prev_row, prev_qb);   // the last task's group
  __builtin_amdgcn_s_waitcnt(0);                           // the last task's Q reloads
}

template <int KC>
__global__ __launch_bounds__(64 * kAW) void tri_attn_kernel(const TriAttnArgs a) { tri_attn_body<false, false, KC>(a); }

__global__ __launch_bounds__(64 * kAW) void tri_ibs_tile_attn_kernel(const TriAttnArgs a) { tri_attn_body<true, false>(a); }

__global__ __launch_bounds__(64 * kAW) void tri_attn_fused_kernel(const TriAttnArgs a) { tri_attn_body<false, true>(a); }

// (row, head) pairs flagged by the attention kernel (a weight sum out of range) of attention row r:
// recomputed with an exact two-pass softmax (maximum first, then weights 2^(s - max)) in fp32 from
// the same Q, K, V^T and bias operands, one query per thread of a 256-thread workgroup; each flag
// is cleared afterwards.
template <int KC = 2>
__device__ void tri_exact_head(const TriAttnArgs& a, int r, int h, int tid) {
  constexpr int D = 16 * KC;
  const int N = a.N, NP = a.NP, H = a.H;
  auto slot_dim = [](int hf, int kk, int t) { return 16 * kk + 8 * (t >> 2) + 4 * hf + (t & 3); };
  {
    if (a.flags[r * H + h] == 0) return;                 // same address for every thread: uniform
    for (int i = tid; i < N; i += 256) {
      // q.k is invariant under the common dim permutation of the Q / K layouts: dot in storage order
      float q[D];
#pragma unroll
      for (int c = 0; c < 2 * KC; ++c) {
        const u32x4 v = ld16(a.q + ql_off<KC>(r, h, H, NP, i, c >> 1, c & 1));
#pragma unroll
        for (int e = 0; e < 4; ++e) { q[8 * c + 2 * e] = bflo(v[e]); q[8 * c + 2 * e + 1] = bfhi(v[e]); }
      }
      auto logit = [&](int j) {
        float s = bf2f(a.bias[bias_off(h, i, j, NP)]);
#pragma unroll
        for (int c = 0; c < 2 * KC; ++c) {
          const u32x4 v = ld16(a.k + ql_off<KC>(r, h, H, NP, j, c >> 1, c & 1));
#pragma unroll
          for (int e = 0; e < 4; ++e) s += q[8 * c + 2 * e] * bflo(v[e]) + q[8 * c + 2 * e + 1] * bfhi(v[e]);
        }
        return s;
      };
      float m = -INFINITY;
      for (int j = 0; j < N; ++j) m = fmaxf(m, logit(j));
      float l = 0.f, acc[D];
#pragma unroll
      for (int d = 0; d < D; ++d) acc[d] = 0.f;
      for (int j = 0; j < N; ++j) {
        const float w = exp2f(logit(j) - m);
        l += w;
        // V^T piece of key j: chunk j/16, lane half (j/4)%2, element 4((j%16)/8) + j%4
        const int c16 = j >> 4, hf = (j >> 2) & 1, t = 4 * ((j & 15) >> 3) + (j & 3);
#pragma unroll
        for (int d = 0; d < D; ++d) acc[d] += w * bf2f(a.vt[vl_off<KC>(r, h, H, NP, c16, hf, d) + t]);
      }
      const float inv = 1.0f / l;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
        for (int kk = 0; kk < KC; ++kk) {
          uint32_t w[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            w[e] = pack_bf2(acc[slot_dim(hf, kk, 2 * e)] * inv, acc[slot_dim(hf, kk, 2 * e + 1)] * inv);
          st16(a.o + o_off<KC>(h, r, i, hf, kk, N, NP), u32x4{w[0], w[1], w[2], w[3]});
        }
      }
    }
    __syncthreads();                                     // every thread has read the flag
    if (tid == 0) a.flags[r * H + h] = 0;
  }
}
__device__ void tri_exact_heads(const TriAttnArgs& a, int r, int tid) {
  for (int h = 0; h < a.H; ++h) tri_exact_head(a, r, h, tid);
}

// ---------------------------------------------------------------------------------------
// Rows the attention kernel cannot finish on its fast path, per (attention row, head) item, the
// items dealt over a fixed grid (a launch of one workgroup per row cost ~4.6 us when every row
// was a no-op):
//  * rows whose token is masked (seq[r] == 0): every logit of the row is masked, so the
//    reference's softmax is uniform over the N keys: o = mean_k V[r, k] (gated later, like
//    every other row).  Keys past N hold V = 0.
//  * (row, head) pairs flagged by tri_attn_kernel (a weight sum out of range): recomputed with
//    an exact two-pass softmax (maximum first, then weights 2^(s - max)) in fp32 from the same
//    Q, K, V^T and bias operands, one query per thread; the flag is cleared afterwards.
// ---------------------------------------------------------------------------------------
constexpr int kFixupGrid = 512;       // workgroups of tri_fixup_kernel (items strided over them)
template <int KC>
__global__ __launch_bounds__(256) void tri_fixup_kernel(const TriAttnArgs a) {
  constexpr int D = 16 * KC, NPART = 256 / D;
  const int H = a.H, tid = threadIdx.x, N = a.N, NP = a.NP, items = N * H;
  // stored slot (lane half hf, k-chunk kk, element t) of a head's D outputs -> dim of V^T
  auto slot_dim = [](int hf, int kk, int t) { return 16 * kk + 8 * (t >> 2) + 4 * hf + (t & 3); };
  __shared__ float part[NPART][D];
  __shared__ float mean[D];
  __shared__ int list[256];
  __shared__ int nlist;
  // this workgroup's items are blockIdx.x + k gridDim.x; 256 of them are checked at once, one per
  // thread (checked one after another, each a dependent load, a no-op launch took 9 us)
  const int K = (items - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
  for (int k0 = 0; k0 < K; k0 += 256) {
    if (tid == 0) nlist = 0;
    __syncthreads();
    {
      const int k = k0 + tid, item = (int)blockIdx.x + k * (int)gridDim.x;
      if (k < K && (a.seq[item / H] == 0 || (!a.sparse && a.flags[item] != 0))) list[atomicAdd(&nlist, 1)] = item;
    }
    __syncthreads();
    const int n = nlist;
    for (int w = 0; w < n; ++w) {                          // (row r, head hb)
      const int item = list[w], r = item / H, hb = item - r * H;
      if (a.seq[r] != 0) {                               // a flagged (row, head): exact recompute
        tri_exact_head<KC>(a, r, hb, tid);
        continue;
      }
      // head hb of a masked row.  Sum over the keys: thread (part p, dim d), part p of the 16-key
      // chunks, all of its loads in flight; then the mean, and the N queries' o of the head.
      // (One workgroup per row, all heads, took 8.5 us for the 38 padded rows of N = 384: a
      // single workgroup's load, reduce and store chain per row is the whole kernel.)
      {
        const int d = tid % D, pp = tid / D, nc = NP / 16;
        float s0 = 0.f, s1 = 0.f;
        for (int c0 = pp; c0 < nc; c0 += NPART * 4) {    // chunks c0 + NPART u, u < 4: all loads issued together
          u32x4 v[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int c16 = c0 + NPART * (u >> 1);
            v[u] = c16 < nc ? ld16(a.vt + vl_off<KC>(r, hb, H, NP, c16, u & 1, d)) : u32x4{0, 0, 0, 0};
          }
#pragma unroll
          for (int u = 0; u < 8; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) { s0 += bflo(v[u][e]); s1 += bfhi(v[u][e]); }
        }
        part[pp][d] = s0 + s1;
      }
      __syncthreads();
      if (tid < D) {
        float t = 0.f;
#pragma unroll
        for (int q = 0; q < NPART; ++q) t += part[q][tid];
        mean[tid] = t / (float)N;
      }
      __syncthreads();
      // one (query, lane half) per thread: 16 dims in epilogue order; consecutive threads write
      // consecutive queries of one piece
      for (int t = tid; t < N * 2; t += 256) {
        const int i = t % N, hf = t / N;
#pragma unroll
        for (int kk = 0; kk < KC; ++kk) {
          uint32_t wv[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) wv[e] = pack_bf2(mean[slot_dim(hf, kk, 2 * e)], mean[slot_dim(hf, kk, 2 * e + 1)]);
          st16(a.o + o_off<KC>(hb, r, i, hf, kk, N, NP), u32x4{wv[0], wv[1], wv[2], wv[3]});
        }
      }
      __syncthreads();                                   // mean is read: the next item may refill it
    }
    __syncthreads();                                     // nlist is read
  }
}

// Rows the fused epilogue left to this kernel (a head of the row was flagged): those heads are
// recomputed exactly, as tri_fixup_kernel does, then the row's output is written (gate, output
// projection, residual) for all its queries.  Grid-strided over the rows; also clears the group
// counts, the marks and (through the recompute) the flags for the next call.
__global__ __launch_bounds__(256) void tri_post_kernel(const TriAttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t sW[kPC * kWP];
  __shared__ __attribute__((aligned(16))) uint16_t sG[kPC * kWP];
  __shared__ __attribute__((aligned(16))) float sGoff[kPC];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = lane >> 5, li = lane & 31;
  const int N = a.N, NP = a.NP;
  for (int f = blockIdx.x * 256 + tid; f < a.groups; f += gridDim.x * 256) a.ctr[f] = 0;
  bool staged = false;
  for (int r = blockIdx.x; r < N; r += gridDim.x) {
    if (a.defer[r] == 0) continue;                       // same address for every thread: uniform
    if (!staged) {
      stage_out_weights<256>(sW, sG, sGoff, a.wo, a.wg, a.goff, tid);
      staged = true;
    }
    tri_exact_heads(a, r, tid);
    // the recomputed o rows are read by other waves below: __syncthreads waits only for LDS
    // traffic, so the global stores are waited for explicitly first
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int ib = wave; ib * 32 < N; ib += 4) {
      const int i = ib * 32 + li;
      const bool ok = i < N;
      const int64_t p = a.transpose ? (int64_t)(ok ? i : 0) * N + r : (int64_t)r * N + (ok ? i : 0);
      u32x4 on[8], zn[8];
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        on[kk] = ok ? ld16(a.o + o_off(kk >> 1, r, i, kk & 1, half, N, NP)) : u32x4{0, 0, 0, 0};
        zn[kk] = ok ? ld16(a.z + p * kPC + 8 * half + 16 * kk) : u32x4{0, 0, 0, 0};
      }
      bf16x8 xg[8];
      uint32_t zr[8][2][2];                                  // unused: the residual is re-read below
      out_gate(on, zn, ok, false, sG, sGoff, lane, xg, zr);
      const uint16_t* zq = a.z + p * kPC + 4 * half;
      out_proj(xg, a.add_residual, sW, lane,
               [&](int nb, int c) { return ok ? *reinterpret_cast<const u32x2*>(zq + 32 * nb + 8 * c) : u32x2{0, 0}; },
               [&](int nb, int c, u32x2 v) {
                 if (ok) *reinterpret_cast<u32x2*>(a.out + p * kPC + 32 * nb + 8 * c + 4 * half) = v;
               });
    }
    __syncthreads();                                     // every thread has read the mark
    if (tid == 0) a.defer[r] = 0;
  }
}

// ---------------------------------------------------------------------------------------
// IBS block-sparse attention (head dim 32 layouts; the projection, fix-up and output stages are
// the dense path's).  Blocks of 32 queries x 32 keys; per (row, head, query tile) S slots of
// (key block, weight).  The sampler:
//   mass of key block b = sum over its valid keys of 2^(qbar . k_j + bbar_j)   (log2 units)
//   qbar, bbar: the tile's mean query and mean bias over its queries (i < N)
//   valid block: one with at least one valid key (whatever its mass)
//   at most S valid blocks: all of them, weight 1 (the dense attention, exactly)
//   else static blocks -- descending mass (ties: lower index), until the mass reaches t_prob, at
//   most S - R -- weight 1; then R draws with replacement from the next blocks up to mass tr_prob,
//   proposal q ~ max(p / M_cand, u_prob) (uniform if M_cand = 0); a block drawn c times gets
//   weight c / (R q)
//   draws: SplitMix64 hash of (seed, batch, row, head, tile, draw), 24 bits -> [0, 1)
// The attention: o_i = sum_s w_s sum_{j in b_s} 2^(s_ij) v_j / sum_s w_s sum_{j in b_s} 2^(s_ij),
// with an exact running maximum.
// ---------------------------------------------------------------------------------------
constexpr int kIbsMaxBlocks = 256;    // key blocks: N <= 8192 (the sampler's LDS: 256 T bytes)
constexpr int kIbsMaxSamples = 64;

struct IbsArgs {
  int N, NP, H, T, S, R, transpose;
  float t_prob, tr_prob, u_prob;
  unsigned long long seed;
  const uint16_t *q, *k, *vt, *bias;
  const uint8_t* seq;
  float* bmean;                       // tile-mean bias (log2 units), ibs_bmean_off order; -inf for keys
                                      // past N or masked (no valid row attends them) and tiles past T
  int32_t* index; float* weight;      // [N][H][T][S]
  uint16_t* o;                        // o_off blocks (per head, attention row, 32 queries), as the dense stage writes them
  const uint8_t* flags;               // (row, head) pairs the tile kernel flagged, for tri_ibs_flagged_kernel
};

__device__ __forceinline__ unsigned long long ibs_mix64(unsigned long long x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// The hash of (seed, batch 0, row, head, tile): the part of a draw's hash all its draws share.
__device__ __forceinline__ unsigned long long ibs_tile_hash(unsigned long long seed, int row, int head, int tile) {
  unsigned long long x = ibs_mix64(seed);
  x = ibs_mix64(x ^ 0ull);                                   // batch 0
  x = ibs_mix64(x ^ (unsigned long long)(unsigned)row);
  x = ibs_mix64(x ^ (unsigned long long)(unsigned)head);
  return ibs_mix64(x ^ (unsigned long long)(unsigned)tile);
}
// Uniform in [0, 1) of draw `draw`: 24 bits of mix64(tile hash ^ draw).
__device__ __forceinline__ float ibs_uniform(unsigned long long tile_hash, int draw) {
  const unsigned long long x = ibs_mix64(tile_hash ^ (unsigned long long)(unsigned)draw);
  return (float)(x >> 40) * (1.0f / 16777216.0f);
}

// Tile-mean bias of (head h, tile t, key j) at [h][t / 32][key block j / 32][quad][t % 32][j % 4]
// with quad = 2 ((j % 32) / 8) + (j / 4) % 2: the sampler's lane (hf, li) seeds its S^T registers
// 4u .. 4u + 3 (keys 32 b + 8u + 4 hf + 0..3) of tile 32 g + li from one 16-byte load, and the 32
// lanes of a half read 512 contiguous bytes.
__host__ __device__ __forceinline__ int64_t ibs_bmean_off(int h, int G, int KB, int t, int j) {
  const int q4 = 2 * ((j & 31) >> 3) + ((j >> 2) & 1);
  return (((((int64_t)h * G + (t >> 5)) * KB + (j >> 5)) * 8 + q4) * 32 + (t & 31)) * 4 + (j & 3);
}

// Tile-mean bias: one thread per (head, tile, key), in ibs_bmean_off order.  A key past N or
// masked gets -inf: the sampler's logits then drop it with no per-key mask test (in a row with
// seq[r] = 1 the valid keys are those with seq[j] = 1; masked rows are not sampled); tiles past T
// (the last group's idle lanes) get -inf as well.
__global__ __launch_bounds__(256) void tri_ibs_bias_mean_kernel(const IbsArgs a) {
  const int KB = a.T, G = (a.T + 31) >> 5;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)a.H * G * KB * 1024) return;
  const int c = (int)(idx & 3), tl = (int)((idx >> 2) & 31), q4 = (int)((idx >> 7) & 7);
  const int64_t rest = idx >> 10;                            // (h, g, key block)
  const int b = (int)(rest % KB), g = (int)((rest / KB) % G), h = (int)(rest / ((int64_t)KB * G));
  const int t = 32 * g + tl, j = 32 * b + 8 * (q4 >> 1) + 4 * (q4 & 1) + c;
  if (t >= a.T || j >= a.N || a.seq[j] == 0) { a.bmean[idx] = -INFINITY; return; }
  const int js = (j & ~63) + bias_pos64(j & 63);
  const int i0 = 32 * t, i1 = min(a.N, i0 + 32);
  float sum = 0.f;
  for (int i = i0; i < i1; ++i) sum += bf2f(a.bias[bias_off_stored(h, i, js, a.NP)]);
  a.bmean[idx] = sum / (float)(i1 - i0);
}

// The sampler: one workgroup of 4 waves per (row r, head h, group of 32 query tiles); lane
// (half, li) of every wave holds tile 32 g + li.  The tile sums of the query are read a whole
// 2 KB tile at a time and reduced across lanes; block logits S^T = K . qbar^T on the MFMA with the
// mean split into two bf16 terms (hi + lo: about 16 significant bits), seeded with the tile-mean
// bias; per block the log2 mass max + log2(sum 2^(x - max)) over its valid keys.  Wave w takes
// the key blocks b = w mod 4; for the ranking lane (hf, li) of wave w takes blocks b = w + 4 hf
// mod 8, writing each block's mass 2^(l2 - M) at its rank.  Lane (0, li) of wave 0 then selects
// tile li's blocks with running sums over those masses and the draw probabilities, each
// computed once.  LDS: log2 masses [KB][32] (later the draw probabilities), order | count << 16
// [KB][32], masses by rank [KB][32], and first, in the same bytes, the tile query sums
// [32 tiles][4 pieces][8 dims].
constexpr int kIbsIndexWaves = 4;

// Sum over the 16 lanes of a DPP row, in every lane of it: mirror, half mirror, then the two
// quad permutations pair each lane with the other 15.
__device__ __forceinline__ float row16_sum(float x) {
  auto dpp = [](float v, auto ctrl) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), decltype(ctrl)::value, 0xF, 0xF, true));
  };
  x += dpp(x, std::integral_constant<int, 0x140>{});       // row_mirror
  x += dpp(x, std::integral_constant<int, 0x141>{});       // row_half_mirror
  x += dpp(x, std::integral_constant<int, 0x1B>{});        // quad_perm [3, 2, 1, 0]
  x += dpp(x, std::integral_constant<int, 0xB1>{});        // quad_perm [1, 0, 3, 2]
  return x;
}

__global__ __launch_bounds__(64 * kIbsIndexWaves) __attribute__((amdgpu_waves_per_eu(8))) void tri_ibs_index_kernel(const IbsArgs a) {
  extern __shared__ float ibs_lds[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, half = lane >> 5, li = lane & 31;
  const int N = a.N, NP = a.NP, H = a.H, T = a.T, KB = a.T, S = a.S;
  const int G = (T + 31) >> 5;
  // the grid is N * H * G.  Workgroup i runs on XCD i mod 8: tasks are dealt so that each XCD
  // takes a contiguous run of them, and the G tile groups of a (row, head), which read the same
  // keys, meet in one L2
  const int ntask = N * H * G, per = ntask >> 3;
  const int task = (int)blockIdx.x < 8 * per ? (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3) : (int)blockIdx.x;
  const int g = task % G, h = (task / G) % H, r = task / (G * H);
  const int t = 32 * g + li, tc = min(t, T - 1);            // tc: operand tile of idle lanes
  const bool owner = wave == 0 && half == 0 && t < T;        // writes tile t's maps
  int32_t* iout = a.index + (((int64_t)r * H + h) * T + tc) * S;
  float* wout = a.weight + (((int64_t)r * H + h) * T + tc) * S;
  float* lm = ibs_lds;
  int* ord = reinterpret_cast<int*>(ibs_lds + KB * 32);
  float* smass = ibs_lds + 2 * KB * 32;                      // masses in rank order
  int filled = 0;
  if (a.seq[r] != 0) {                                       // uniform over the workgroup
    // tile sums of the query: wave w sums tiles 32 g + 8 w .. + 7, one 2 KB tile (4 pieces of 32
    // positions x 8 dims) per step: lane (row pc, p) adds positions p and p + 16 of piece pc, its
    // 16-lane row then reduces (DPP); lane p = 0 stores the piece's 8 sums to qsum[tile][piece]
    float* qsum = ibs_lds;                                   // [32][4][8], before lm / ord / smass
    {
      const int pc = lane >> 4, p = lane & 15;
#pragma unroll 2
      for (int it = 0; it < 8; ++it) {
        const int tl = 8 * wave + it, tq = min(32 * g + tl, T - 1);
        const uint16_t* qt = a.q + ql_off(r, h, H, NP, 32 * tq, 0, 0) + pc * 256 + p * 8;
        const u32x4 v0 = ld16(qt), v1 = ld16(qt + 128);
        float sv[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sv[2 * e] = bflo(v0[e]) + bflo(v1[e]);
          sv[2 * e + 1] = bfhi(v0[e]) + bfhi(v1[e]);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) sv[e] = row16_sum(sv[e]);
        if (p == 0) {
          f32x4* dst = reinterpret_cast<f32x4*>(qsum + (tl * 4 + pc) * 8);
          dst[0] = f32x4{sv[0], sv[1], sv[2], sv[3]};
          dst[1] = f32x4{sv[4], sv[5], sv[6], sv[7]};
        }
      }
    }
    __syncthreads();
    float qs[2][8];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const f32x4* src = reinterpret_cast<const f32x4*>(qsum + (li * 4 + 2 * kk + half) * 8);
      const f32x4 x0 = src[0], x1 = src[1];
#pragma unroll
      for (int e = 0; e < 4; ++e) { qs[kk][e] = x0[e]; qs[kk][4 + e] = x1[e]; }
    }
    __syncthreads();                                         // qsum read: lm may be written
    const float qinv = 1.0f / (float)(min(N, 32 * tc + 32) - 32 * tc);   // queries past N hold 0
    bf16x8 qh[2], ql[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = qs[kk][e] * qinv;
        const __bf16 hv = (__bf16)v;
        qh[kk][e] = hv;
        ql[kk][e] = (__bf16)(v - (float)hv);
      }
    const float* bm = a.bmean + ibs_bmean_off(h, G, KB, t, 0);   // tile t's column (past T: -inf)
    // block b's operands: K (two k-chunks) and the tile-mean bias of its 16 keys in this lane
    auto load_block = [&](int b, u32x4 (&kv)[2], f32x16& bv) {
      const int j = 32 * b + li;
      kv[0] = ld16(a.k + ql_off(r, h, H, NP, j, 0, half));
      kv[1] = ld16(a.k + ql_off(r, h, H, NP, j, 1, half));
      const float* bp = bm + (int64_t)b * 8 * 128 + half * 128;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(bp + u * 256);   // quad 2u + hf
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[4 * u + e] = v[e];
      }
    };
    for (int b = wave; b < KB; b += kIbsIndexWaves) {
      u32x4 kn[2];
      f32x16 sc;                                             // seeded with the tile-mean bias
      load_block(b, kn, sc);
      const bf16x8 k0 = as_bf16x8(kn[0]), k1 = as_bf16x8(kn[1]);
      sc = mfma32(k0, qh[0], sc);
      sc = mfma32(k1, qh[1], sc);
      sc = mfma32(k0, ql[0], sc);
      sc = mfma32(k1, ql[1], sc);
      // invalid keys hold -inf (their tile-mean bias): they add exactly 0.  The hardware exp2
      // (no denormal range reduction): a term below 2^-126 is lost against the block maximum's 1
      float mx = -INFINITY;
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, sc[e]);
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      float sum = 0.f;
      if (mx != -INFINITY) {
#pragma unroll
        for (int e = 0; e < 16; ++e) sum += __builtin_amdgcn_exp2f(sc[e] - mx);
      }
      sum += __shfl_xor(sum, 32);
      const float l2 = mx + log2f(sum);
      if (half == 0) lm[b * 32 + li] = (mx == -INFINITY || l2 != l2) ? -INFINITY : l2;   // NaN: no block
    }
    __syncthreads();
    float M = -INFINITY;
    int nvalid = 0;
    for (int b = 0; b < KB; ++b) {
      const float v = lm[b * 32 + li];
      M = fmaxf(M, v);
      nvalid += v != -INFINITY;
    }
    // descending mass, ties: lower index first; blocks without valid keys are not ranked
    if (nvalid > S) {
      // half hf ranks block b0 + 4 hf; the loop bounds stay wave-uniform: blocks c < b0 count when
      // at least as heavy (ties: the lower index first), c > b0 + 4 when heavier
      const int w0 = __builtin_amdgcn_readfirstlane(wave);
      for (int b0 = w0; b0 < KB; b0 += 2 * kIbsIndexWaves) {
        const int b = b0 + kIbsIndexWaves * half;
        const float v = b < KB ? lm[b * 32 + li] : -INFINITY;
        int rank = 0;
#pragma unroll 8
        for (int c = 0; c < b0; ++c) rank += lm[c * 32 + li] >= v;
        const int c1 = min(b0 + kIbsIndexWaves + 1, KB);
        for (int c = b0; c < c1; ++c) {
          const float u = lm[c * 32 + li];
          rank += (u > v) || (u == v && c < b);
        }
#pragma unroll 8
        for (int c = c1; c < KB; ++c) rank += lm[c * 32 + li] > v;
        if (v != -INFINITY) {
          ord[rank * 32 + li] = b;
          smass[rank * 32 + li] = exp2f(v - M);
        }
      }
    }
    __syncthreads();
    if (owner) {
      if (nvalid <= S) {                                     // every valid block, weight 1
        for (int b = 0; b < KB; ++b)
          if (lm[b * 32 + li] != -INFINITY) { iout[filled] = b; wout[filled] = 1.f; ++filled; }
      } else {
        auto mass = [&](int k) { return smass[k * 32 + li]; };
        float total = 0.f;
        for (int k = 0; k < nvalid; ++k) total += mass(k);
        const float inv = 1.0f / total;
        int ns = 0;
        float cum = 0.f;
        while (ns < nvalid && cum < a.t_prob && ns < S - a.R) { cum += mass(ns) * inv; ++ns; }
        int nc = 0;
        while (ns + nc < nvalid && cum < a.tr_prob) { cum += mass(ns + nc) * inv; ++nc; }
        for (int k = 0; k < ns; ++k) { iout[k] = ord[k * 32 + li]; wout[k] = 1.f; }
        filled = ns;
        if (nc > 0 && a.R > 0) {
          float mc = 0.f;
          for (int c = 0; c < nc; ++c) mc += mass(ns + c) * inv;
          // the draw probabilities q_c = raw_c / sum raw once, in the (now free) log2-mass
          // column of this tile
          float* qc = lm;
          float zr = 0.f;
          for (int c = 0; c < nc; ++c) {
            const float rc = mc > 0.f ? fmaxf(mass(ns + c) * inv / mc, a.u_prob) : 1.0f;
            qc[c * 32 + li] = rc;
            zr += rc;
          }
          for (int c = 0; c < nc; ++c) qc[c * 32 + li] = qc[c * 32 + li] / zr;
          const unsigned long long th = ibs_tile_hash(a.seed, r, h, t);
          for (int d = 0; d < a.R; ++d) {
            const float uu = ibs_uniform(th, d);
            float acc = 0.f;
            int pick = nc - 1;
            for (int c = 0; c < nc; ++c) {
              acc += qc[c * 32 + li];
              if (uu < acc) { pick = c; break; }
            }
            ord[(ns + pick) * 32 + li] += 1 << 16;
          }
          for (int c = 0; c < nc; ++c) {
            const int cnt = ord[(ns + c) * 32 + li] >> 16;
            if (cnt == 0) continue;
            iout[filled] = ord[(ns + c) * 32 + li] & 0xFFFF;
            wout[filled] = (float)cnt / ((float)a.R * qc[c * 32 + li]);
            ++filled;
          }
        }
      }
    }
  }
  if (owner)
    for (int s = filled; s < S; ++s) { iout[s] = -1; wout[s] = 0.f; }
}

// Exact sparse attention: one wave per (row, head, query tile); per selected block the S^T MFMAs
// seeded with the bias, an exact running maximum, weights w 2^(s - m) as bf16, P.V on the MFMA.
// Output in the dense stage's o layout, so the output stage is shared.  Masked rows are left to
// the fix-up kernel.  It recomputes the (row, head) pairs tri_ibs_tile_attn_kernel flagged (a
// weight sum out of range of its fixed reference point), or every row where that kernel's
// per-wave table cannot hold the key blocks (N > 4096).
__device__ void ibs_exact_tile(const IbsArgs& a, int r, int h, int t) {
  const int lane = threadIdx.x & 63, half = lane >> 5, li = lane & 31;
  const int64_t task = ((int64_t)r * a.H + h) * a.T + t;
  const int N = a.N, NP = a.NP, H = a.H;
  const int i = 32 * t + li;                                 // this lane's query (< NP)
  bf16x8 qb[2];
  const uint16_t* qp = a.q + ql_off(r, h, H, NP, i, 0, half);
  qb[0] = as_bf16x8(ld16(qp));
  qb[1] = as_bf16x8(ld16(qp + 512));
  f32x16 o;
#pragma unroll
  for (int e = 0; e < 16; ++e) o[e] = 0.f;
  float m = -INFINITY, l = 0.f;
  const int32_t* idx = a.index + task * a.S;
  const float* wts = a.weight + task * a.S;
  for (int s = 0; s < a.S; ++s) {
    const int b = idx[s];                                    // same address in every lane: uniform
    const float w = wts[s];
    // unused slot: index out of range or weight <= 0 (the tile kernel's table skips the same)
    if (b < 0 || b >= a.T || !(w > 0.f)) continue;
    bf16x8 kr[2], vr[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) kr[kk] = as_bf16x8(ld16(a.k + ql_off(r, h, H, NP, 32 * b + li, kk, half)));
#pragma unroll
    for (int j = 0; j < 2; ++j) vr[j] = as_bf16x8(ld16(a.vt + vl_off(r, h, H, NP, 2 * b + j, half, li)));
    // bias of query i for keys 8(e/4) + 4 half + e%4 of the block: stored positions
    // 32 (b & 1) + 16 half + e of its 64-key tile, two pieces of 8
    const int js = 64 * (b >> 1) + 32 * (b & 1) + 16 * half;
    const u32x4 b0 = ld16(a.bias + bias_off_stored(h, i, js, NP)), b1 = ld16(a.bias + bias_off_stored(h, i, js + 8, NP));
    f32x16 sd;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sd[2 * e] = bflo(b0[e]); sd[2 * e + 1] = bfhi(b0[e]);
      sd[8 + 2 * e] = bflo(b1[e]); sd[8 + 2 * e + 1] = bfhi(b1[e]);
    }
    const f32x16 sc = mfma32(kr[1], qb[1], mfma32(kr[0], qb[0], sd));
    float bmx = sc[0];
#pragma unroll
    for (int e = 1; e < 16; ++e) bmx = fmaxf(bmx, sc[e]);
    bmx = fmaxf(bmx, __shfl_xor(bmx, 32));
    const float mn = fmaxf(m, bmx);
    const float alpha = m == -INFINITY ? 0.f : fast_exp2(m - mn);
#pragma unroll
    for (int e = 0; e < 16; ++e) o[e] *= alpha;
    l *= alpha;
    m = mn;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      bf16x8 pb;
#pragma unroll
      for (int q2 = 0; q2 < 4; ++q2) {
        const bf16x2 pw = cvt_bf2(w * fast_exp2(sc[8 * j + 2 * q2] - mn), w * fast_exp2(sc[8 * j + 2 * q2 + 1] - mn));
        pb[2 * q2] = pw[0];
        pb[2 * q2 + 1] = pw[1];
        l += (float)pw[0] + (float)pw[1];
      }
      o = mfma32(vr[j], pb, o);
    }
  }
  const float lt = l + __shfl_xor(l, 32);
  if (i >= N) return;
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    uint32_t w4[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) w4[e] = pack_bf2(o[8 * kk + 2 * e] * inv, o[8 * kk + 2 * e + 1] * inv);
    st16(a.o + o_off(h, r, i, half, kk, N, NP), u32x4{w4[0], w4[1], w4[2], w4[3]});
  }
}

// Every (row, head, query tile) of the valid rows, one wave each (N > 4096: the attention itself).
__global__ __launch_bounds__(256) void tri_ibs_attn_kernel(const IbsArgs a) {
  const int64_t task = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (task >= (int64_t)a.N * a.H * a.T) return;
  const int t = (int)(task % a.T), h = (int)((task / a.T) % a.H), r = (int)(task / ((int64_t)a.T * a.H));
  if (a.seq[r] == 0) return;
  ibs_exact_tile(a, r, h, t);
}

// The (row, head) pairs the tile kernel flagged: (row, head) items dealt over a fixed grid, a
// workgroup's items checked at once (one per thread), its 4 waves then taking the query tiles of
// each flagged pair.  (One wave per (row, head, tile) that checked its pair's flag and mostly
// returned took 51 us at N = 1536 with nothing flagged: 295k waves dispatched for nothing.)
constexpr int kIbsFlaggedGrid = 1024;
__global__ __launch_bounds__(256) void tri_ibs_flagged_kernel(const IbsArgs a) {
  __shared__ int list[256];
  __shared__ int nlist;
  const int tid = threadIdx.x, wave = tid >> 6, items = a.N * a.H;
  const int K = (items - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
  for (int k0 = 0; k0 < K; k0 += 256) {
    if (tid == 0) nlist = 0;
    __syncthreads();
    {
      const int k = k0 + tid, item = (int)blockIdx.x + k * (int)gridDim.x;
      if (k < K && a.seq[item / a.H] != 0 && a.flags[item] != 0) list[atomicAdd(&nlist, 1)] = item;
    }
    __syncthreads();
    const int n = nlist;
    for (int w = 0; w < n; ++w) {
      const int item = list[w], r = item / a.H, h = item - r * a.H;
      for (int t = wave; t < a.T; t += 4) ibs_exact_tile(a, r, h, t);
    }
    __syncthreads();                                       // nlist and list are read
  }
}

// ---------------------------------------------------------------------------------------
// Generic path (any head dim): LN -> linear -> strided attention -> linear
// ---------------------------------------------------------------------------------------
struct TriWs {
  uint16_t* xhat;   // [P, C]
  uint16_t* y;      // [P, 4HD]  q | k | v | g
  uint16_t* bias;   // [H, P]
  uint16_t* o;      // [P, HD]
  size_t bytes;
};

// The fast paths: head dim 32 with C = 128 (the trunk; also the block-sparse mode) and head dim
// 16 with C = 64 (the template stack), four heads each.
bool fast_path(int32_t C, int32_t H, int32_t D) { return C == kPC && D == 32 && H * D == kPC; }
bool fast16_path(int32_t C, int32_t H, int32_t D) { return C == TriDims<1>::C && D == 16 && H == 4; }

TriWs carve(void* base, int32_t N, int32_t C, int32_t H, int32_t D) {
  const size_t P = (size_t)N * N, HD = (size_t)H * D;  TriWs w{};
  char* p = (char*)base;
  size_t off = 0;
  w.xhat = (uint16_t*)(p + off); off += round_up(P * C * 2);
  w.y = (uint16_t*)(p + off); off += round_up(P * 4 * HD * 2);
  w.bias = (uint16_t*)(p + off); off += round_up(P * H * 2);
  w.o = (uint16_t*)(p + off); off += round_up(P * HD * 2);
  w.bytes = off;
  return w;
}
}  // namespace

extern "C" size_t sf_hip_triangle_workspace_bytes(int32_t N, int32_t C, int32_t H, int32_t D) {
  if (N <= 0 || C <= 0 || H <= 0 || D <= 0) return 0;
  if (fast_path(C, H, D)) return carve_fast<2>(nullptr, N, H).bytes;
  if (fast16_path(C, H, D)) return carve_fast<1>(nullptr, N, H).bytes;
  return carve(nullptr, N, C, H, D).bytes;
}

namespace {
// Persistent launch size: enough waves to cover every CU a few times, each wave walking a
// contiguous run of items so that neighbouring waves touch neighbouring memory.
int persistent_groups(int items, int* items_per_wave) {
  const int target_waves = 256 * 4 * 2;               // 256 CUs x 4 SIMDs x 2 waves
  int ipw = (items + target_waves - 1) / target_waves;
  if (ipw < 1) ipw = 1;
  *items_per_wave = ipw;
  const int waves = (items + ipw - 1) / ipw;
  return (waves + kPWaves - 1) / kPWaves;
}

// Weight sum above which the attention kernel flags a (row, head) for the exact fix-up: 2^100,
// or the caller's smaller positive limit (tests drive the fix-up path with ordinary logits).
float sum_limit(float requested) {
  const float v = 0x1p100f;
  return requested > 0.f && requested <= v ? requested : v;
}

template <int KC>
int triangle_fast(const sf_triangle_args* a, void* workspace, size_t workspace_bytes, hipStream_t st, int stages) {
  using TD = TriDims<KC>;
  const int32_t N = a->N, H = a->H;
  const FastWs ws = carve_fast<KC>(workspace, N, H);
  if (workspace == nullptr || workspace_bytes < ws.bytes) {
    sf_set_error("triangle: workspace too small (%zu < %zu bytes)", workspace_bytes, ws.bytes);
    return 1;
  }
  const int NP = round_np(N);
  if (stages & SF_TRI_STAGE_PROJECT) {
    TriFoldArgs fa{};
    fa.nrows = 4 * H * TD::D + H;
    fa.w = (const uint16_t*)a->w_qkvgb; fa.ln_w = a->ln_w; fa.ln_b = a->ln_b;
    fa.wf = ws.wf; fa.off = ws.off;
    fa.flags = ws.flags; fa.nflags = N * H;
    fa.ctr = ws.ctr; fa.nctr = ws.nctr;
    fa.defer = ws.defer; fa.ndefer = N;
    fa.rgl = ws.rgl; fa.rg = NP / 4; fa.N = N; fa.seq = a->seq_mask;
    hipLaunchKernelGGL(tri_fold_kernel<KC>, dim3(TD::Cols / 4 + 1), dim3(256), 0, st, fa);
    if (int rc = sf_check_launch("tri_fold_kernel")) return rc;

    TriProjArgs pa{};
    pa.N = N; pa.NP = NP; pa.H = H; pa.transpose = a->transpose;
    pa.qscale = (1.0f / sqrtf((float)TD::D)) * SF_LOG2E;
    pa.z = (const uint16_t*)a->z; pa.seq = a->seq_mask;
    pa.wf = ws.wf; pa.off = ws.off;
    pa.q = ws.q; pa.k = ws.k; pa.vt = ws.vt; pa.bias = ws.bias;
    pa.items = NP * (NP / 32);
    const int pgroups = persistent_groups(pa.items, &pa.items_per_wave);
    hipLaunchKernelGGL(tri_proj_kernel<KC>, dim3(pgroups), dim3(64 * kPWaves), 0, st, pa);
    if (int rc = sf_check_launch("tri_proj_kernel")) return rc;
  }

  if (stages & SF_TRI_STAGE_ATTEND) {
    TriAttnArgs aa{};
    aa.N = N; aa.NP = NP; aa.H = H; aa.transpose = a->transpose;
    aa.sum_limit = sum_limit(a->fixup_sum_limit);
    aa.q = ws.q; aa.k = ws.k; aa.vt = ws.vt; aa.bias = ws.bias; aa.seq = a->seq_mask; aa.o = ws.o;
    aa.flags = ws.flags;
    aa.rgl = ws.rgl;                // (the fused kernel ignores it: its epilogue writes every row)
    const int total = ((NP + 32 * kAW - 1) / (32 * kAW)) * (NP / kTR) * H;   // a multiple of 64
    // attention with the gate, output projection and residual in its epilogue: the workgroups
    // of a group's four heads must be resident together on one XCD, so the grid is a multiple of
    // 32 (each XCD's share a multiple of 4) no larger than the resident count
    const int fgrid = std::min(std::min(total, 256),
                               sf_resident_workgroups((const void*)tri_attn_fused_kernel, 64 * kAW) / 32 * 32);
    // (head dim 16: the separate output stage; SF_TRI_STAGE_FUSE is ignored)
    if (KC == 2 && (stages & SF_TRI_STAGE_FUSE) && (stages & SF_TRI_STAGE_OUTPUT) && fgrid >= 32) {
      aa.wo = (const uint16_t*)a->w_o;
      aa.wg = ws.wf + (size_t)12 * 32 * kPC; aa.goff = ws.off + 12 * 32;   // folded gate rows 384..511
      aa.z = (const uint16_t*)a->z; aa.out = (uint16_t*)a->out; aa.add_residual = a->add_residual;
      aa.ctr = ws.ctr; aa.defer = ws.defer; aa.groups = fused_groups(N);
      hipLaunchKernelGGL(tri_attn_fused_kernel, dim3(fgrid), dim3(64 * kAW), 0, st, aa);
      if (int rc = sf_check_launch("tri_attn_fused_kernel")) return rc;
      hipLaunchKernelGGL(tri_post_kernel, dim3(std::min(N, 128)), dim3(256), 0, st, aa);
      return sf_check_launch("tri_post_kernel");
    }
    hipLaunchKernelGGL(tri_attn_kernel<KC>, dim3(std::min(total, 256)), dim3(64 * kAW), 0, st, aa);
    if (int rc = sf_check_launch("tri_attn_kernel")) return rc;
    hipLaunchKernelGGL(tri_fixup_kernel<KC>, dim3(std::min(N * a->H, kFixupGrid)), dim3(256), 0, st, aa);
    if (int rc = sf_check_launch("tri_fixup_kernel")) return rc;
  }
  if (!(stages & SF_TRI_STAGE_OUTPUT)) return 0;

  TriOutArgs oa{};
  oa.N = N; oa.NP = NP; oa.transpose = a->transpose;
  oa.o = ws.o; oa.wo = (const uint16_t*)a->w_o;
  oa.wg = ws.wf + (size_t)3 * TD::C * TD::C; oa.goff = ws.off + 3 * TD::C;   // folded gate rows 3C .. 4C-1
  oa.z = (const uint16_t*)a->z; oa.add_residual = a->add_residual;
  oa.out = (uint16_t*)a->out;
  oa.items = N * ((N + 31) / 32);
  const int ogroups = persistent_groups(oa.items, &oa.items_per_wave);
  hipLaunchKernelGGL(tri_out_kernel<KC>, dim3(ogroups), dim3(64 * kPWaves), 0, st, oa);
  return sf_check_launch("tri_out_kernel");
}
}  // namespace

static int triangle_run(const sf_triangle_args* a, void* workspace, size_t workspace_bytes, void* stream,
                        int stages) {
  if (a == nullptr || a->z == nullptr || a->seq_mask == nullptr || a->ln_w == nullptr ||
      a->w_qkvgb == nullptr || a->w_o == nullptr || a->out == nullptr) {
    sf_set_error("triangle: null pointer argument"); return 1;
  }
  const int32_t N = a->N, C = a->C, H = a->H, D = a->D;
  if (N <= 0 || C <= 0 || H <= 0 || D <= 0 || C % 8 != 0 || D > 64 || (int64_t)H * D > 1024 || (H * D) % 8 != 0) {
    sf_set_error("triangle: unsupported sizes N=%d C=%d H=%d D=%d", N, C, H, D); return 1;
  }
  if (N > 65535) { sf_set_error("triangle: N=%d exceeds the grid limit", N); return 1; }
  if (a->out == a->z) { sf_set_error("triangle: out must not alias z"); return 1; }
  if (fast_path(C, H, D))
    return triangle_fast<2>(a, workspace, workspace_bytes, reinterpret_cast<hipStream_t>(stream), stages);
  if (fast16_path(C, H, D))
    return triangle_fast<1>(a, workspace, workspace_bytes, reinterpret_cast<hipStream_t>(stream), stages);
  if ((stages & SF_TRI_STAGE_ALL) != SF_TRI_STAGE_ALL) {
    sf_set_error("triangle: single stages are available on the fast paths only (C=128, H=4, D=32 or C=64, H=4, "
                 "D=16; given C=%d H=%d D=%d)", C, H, D);
    return 1;
  }
  const TriWs ws = carve(workspace, N, C, H, D);
  if (workspace == nullptr || workspace_bytes < ws.bytes) {
    sf_set_error("triangle: workspace too small (%zu < %zu bytes)", workspace_bytes, ws.bytes); return 1;
  }
  const int64_t P = (int64_t)N * N, HD = (int64_t)H * D;
  int rc;

  sf_layer_norm_args ln{};
  ln.M = P; ln.C = C; ln.eps = 1e-5f;
  ln.x = a->z; ln.x_rs = C;
  ln.gamma = a->ln_w; ln.beta = a->ln_b;
  ln.y = ws.xhat; ln.y_rs = C;
  if ((rc = sf_hip_layer_norm_fwd(&ln, stream))) return rc;

  sf_linear_args pr{};
  pr.M = P; pr.N = (int32_t)(4 * HD + H); pr.K = C;
  pr.x = ws.xhat; pr.x_rs = C; pr.wt = a->w_qkvgb;
  pr.y = ws.y; pr.y_rs = 4 * HD; pr.ycols = (int32_t)(4 * HD);
  pr.tcol0 = (int32_t)(4 * HD); pr.tcols = H; pr.yt = ws.bias; pr.yt_rs = P;
  pr.mul_rows = 1;
  if ((rc = sf_hip_linear_fwd(&pr, stream))) return rc;

  sf_attention_args at{};
  at.B0 = N; at.B1 = 1; at.Q = N; at.K = N; at.H = H; at.D = D; at.Dv = D;
  at.scale = 1.0f / sqrtf((float)D);
  const int64_t rs = 4 * HD;                     // row stride of y
  const int64_t s_row = a->transpose ? rs : (int64_t)N * rs;   // batch row r
  const int64_t s_pos = a->transpose ? (int64_t)N * rs : rs;   // position within the row
  const uint16_t* y = ws.y;
  at.q = y;            at.q_s[0] = s_row; at.q_s[1] = 0; at.q_s[2] = s_pos; at.q_s[3] = D;
  at.k = y + HD;       at.k_s[0] = s_row; at.k_s[1] = 0; at.k_s[2] = s_pos; at.k_s[3] = D;
  at.v = y + 2 * HD;   at.v_s[0] = s_row; at.v_s[1] = 0; at.v_s[2] = s_pos; at.v_s[3] = D;
  at.gate = y + 3 * HD; at.g_s[0] = s_row; at.g_s[1] = 0; at.g_s[2] = s_pos; at.g_s[3] = D;
  at.bias = ws.bias;   at.bias_s[0] = 0; at.bias_s[1] = 0; at.bias_s[2] = P; at.bias_s[3] = N;
  at.mask_q = a->seq_mask; at.mq_s[0] = 1; at.mq_s[1] = 0; at.mq_s[2] = 0;   // row r valid
  at.mask_k = a->seq_mask; at.mk_s[0] = 0; at.mk_s[1] = 0; at.mk_s[2] = 1;   // key k valid
  const int64_t o_row = a->transpose ? HD : (int64_t)N * HD;
  const int64_t o_pos = a->transpose ? (int64_t)N * HD : HD;
  at.out = ws.o; at.o_s[0] = o_row; at.o_s[1] = 0; at.o_s[2] = o_pos; at.o_s[3] = D;
  if ((rc = sf_hip_attention_fwd(&at, stream))) return rc;

  sf_linear_args op{};
  op.M = P; op.N = C; op.K = (int32_t)HD;
  op.x = ws.o; op.x_rs = HD; op.wt = a->w_o;
  if (a->add_residual) { op.residual = a->z; op.r_rs = C; }
  op.mul_rows = 1;
  op.y = a->out; op.y_rs = C;
  return sf_hip_linear_fwd(&op, stream);
}

extern "C" int sf_hip_triangle_attn_fwd(const sf_triangle_args* a, void* workspace, size_t workspace_bytes,
                                        void* stream) {
  return triangle_run(a, workspace, workspace_bytes, stream, SF_TRI_STAGE_ALL);
}

extern "C" int sf_hip_triangle_stage_fwd(const sf_triangle_args* a, int32_t stages, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  if (stages <= 0 || (stages & ~(SF_TRI_STAGE_ALL | SF_TRI_STAGE_FUSE)) || stages == SF_TRI_STAGE_FUSE) {
    sf_set_error("triangle: invalid stage mask %d", stages);
    return 1;
  }
  return triangle_run(a, workspace, workspace_bytes, stream, stages);
}

namespace {
size_t ibs_bmean_offset(int32_t N, int32_t H) { return carve_fast(nullptr, N, H).bytes; }
size_t ibs_ws_bytes(int32_t N, int32_t H) {
  const int T = (N + 31) / 32, G = (T + 31) / 32;
  return ibs_bmean_offset(N, H) + round_up((size_t)H * G * T * 1024 * 4);
}
}  // namespace

extern "C" size_t sf_hip_triangle_ibs_workspace_bytes(int32_t N, int32_t C, int32_t H, int32_t D) {
  if (N <= 0 || !fast_path(C, H, D) || N > 32 * kIbsMaxBlocks) return 0;
  return ibs_ws_bytes(N, H);
}

extern "C" int sf_hip_triangle_attn_ibs_fwd(const sf_triangle_args* a, const sf_ibs_args* p, void* workspace,
                                            size_t workspace_bytes, void* stream) {
  if (a == nullptr || p == nullptr || p->index_map == nullptr || p->weight_map == nullptr) {
    sf_set_error("triangle_ibs: null arguments or maps"); return 1;
  }
  if (!fast_path(a->C, a->H, a->D)) {
    sf_set_error("triangle_ibs: block-sparse attention needs C = 128, D = 32, H = 4 (C=%d H=%d D=%d)", a->C, a->H, a->D);
    return 1;
  }
  if (a->N <= 0 || a->N > 32 * kIbsMaxBlocks) {
    sf_set_error("triangle_ibs: N=%d outside [1, %d]", a->N, 32 * kIbsMaxBlocks); return 1;
  }
  if (p->num_samples < 1 || p->num_samples > kIbsMaxSamples || p->num_rand_blocks < 0 ||
      p->num_rand_blocks > p->num_samples || !(p->t_prob >= 0.f && p->t_prob <= 1.f) ||
      !(p->tr_prob >= 0.f && p->tr_prob <= 1.f) || !(p->u_prob >= 0.f && p->u_prob <= 1.f)) {
    sf_set_error("triangle_ibs: need 1 <= num_samples <= %d, 0 <= num_rand_blocks <= num_samples and "
                 "probabilities in [0, 1]", kIbsMaxSamples);
    return 1;
  }
  if (workspace == nullptr || workspace_bytes < ibs_ws_bytes(a->N, a->H)) {
    sf_set_error("triangle_ibs: workspace of %zu bytes needed, %zu given", ibs_ws_bytes(a->N, a->H), workspace_bytes);
    return 1;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  int rc;
  if ((rc = triangle_run(a, workspace, workspace_bytes, stream, SF_TRI_STAGE_PROJECT))) return rc;
  const FastWs ws = carve_fast(workspace, a->N, a->H);
  IbsArgs ia{};
  ia.N = a->N; ia.NP = round_np(a->N); ia.H = a->H; ia.T = (a->N + 31) / 32;
  ia.S = p->num_samples; ia.R = p->num_rand_blocks; ia.transpose = a->transpose;
  ia.t_prob = p->t_prob; ia.tr_prob = p->tr_prob; ia.u_prob = p->u_prob; ia.seed = p->seed;
  ia.q = ws.q; ia.k = ws.k; ia.vt = ws.vt; ia.bias = ws.bias; ia.seq = a->seq_mask;
  ia.bmean = reinterpret_cast<float*>(static_cast<char*>(workspace) + ibs_bmean_offset(a->N, a->H));
  ia.index = p->index_map; ia.weight = p->weight_map; ia.o = ws.o;
  const int64_t tasks = (int64_t)ia.N * ia.H * ia.T;
  if (p->generate_maps) {
    const int64_t nb = (int64_t)ia.H * ((ia.T + 31) / 32) * ia.T * 1024;
    hipLaunchKernelGGL(tri_ibs_bias_mean_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, st, ia);
    if ((rc = sf_check_launch("tri_ibs_bias_mean_kernel"))) return rc;
    const int groups = (ia.T + 31) / 32;
    const size_t lds = std::max((size_t)3 * ia.T * 32 * 4, (size_t)32 * 4 * 8 * 4);   // <= 96 KB (T <= 256)
    hipLaunchKernelGGL(tri_ibs_index_kernel, dim3((unsigned)(ia.N * ia.H * groups)), dim3(64 * kIbsIndexWaves), lds,
                       st, ia);
    if ((rc = sf_check_launch("tri_ibs_index_kernel"))) return rc;
  }
  TriAttnArgs fa{};
  fa.N = a->N; fa.NP = ia.NP; fa.H = a->H; fa.transpose = a->transpose; fa.sum_limit = sum_limit(a->fixup_sum_limit);
  fa.q = ws.q; fa.k = ws.k; fa.vt = ws.vt; fa.bias = ws.bias; fa.seq = a->seq_mask; fa.o = ws.o; fa.flags = ws.flags;
  fa.index = p->index_map; fa.weight = p->weight_map; fa.T = ia.T; fa.S = ia.S; fa.sparse = 1;
  if (ia.T <= kIbsTabBlocks && ia.NP <= 32 * kIbsTabBlocks) {
    // the tile pipeline with skipped units, then the exact kernel on the rows it flagged
    const int total = ((ia.NP + 32 * kAW - 1) / (32 * kAW)) * (ia.NP / kTR) * a->H;
    hipLaunchKernelGGL(tri_ibs_tile_attn_kernel, dim3(std::min(total, 256)), dim3(64 * kAW), 0, st, fa);
    if ((rc = sf_check_launch("tri_ibs_tile_attn_kernel"))) return rc;
    ia.flags = ws.flags;
  }
  if (ia.flags != nullptr) {
    hipLaunchKernelGGL(tri_ibs_flagged_kernel, dim3((unsigned)std::min(ia.N * ia.H, kIbsFlaggedGrid)), dim3(256), 0, st, ia);
    if ((rc = sf_check_launch("tri_ibs_flagged_kernel"))) return rc;
  } else {
    hipLaunchKernelGGL(tri_ibs_attn_kernel, dim3((unsigned)((tasks + 3) / 4)), dim3(256), 0, st, ia);
    if ((rc = sf_check_launch("tri_ibs_attn_kernel"))) return rc;
  }
  hipLaunchKernelGGL(tri_fixup_kernel<2>, dim3(std::min(a->N * a->H, kFixupGrid)), dim3(256), 0, st, fa);   // masked rows: mean of V
  if ((rc = sf_check_launch("tri_fixup_kernel"))) return rc;
  return triangle_run(a, workspace, workspace_bytes, stream, SF_TRI_STAGE_OUTPUT);
}
