// Gated pair-biased flash attention for gfx950 (generic strided form).
//
// Replaces the Torch math composite of dot_product_attention
// (src/sparsefold/backends/torch/attention/sdpa.py:22-121) and the gate multiply that every
// caller applies to its result (blocks.py:288-289, transformer.py:339-342, :580-583).
//
// Work decomposition: one workgroup = 4 waves = 128 queries of one (batch, head); each wave
// owns 32 queries.  Keys stream through LDS in tiles of 64: K row-major and V transposed
// (keys contiguous, in the slot order the PV MFMA consumes).  Per tile and wave:
//   S^T(64 keys x 32 queries) = K * Q^T       4 x v_mfma_f32_32x32x16_bf16 per 32-dim chunk
//   online softmax in the log2 domain, one query per lane (its 32 keys in registers, the
//   other 32 in lane^32), masked keys -> SF_MASKED_LOGIT, keys past K -> -inf
//   O^T(D x 32 queries) += V^T * P^T          P^T fed from registers as the B operand
// Epilogue: O / l, optional sigmoid gate, bf16 store.
#include <cstdlib>

#include <type_traits>

#include "sf_common.h"

namespace {

constexpr int kQB = 128;  // queries per workgroup
constexpr int kKT = 64;   // keys per tile

__device__ __forceinline__ int vt_pos(int r) {
  // position of tile key r in the transposed V tile: 16-key chunk, then lane half, then slot
  const int c2 = r >> 4, k16 = r & 15;
  const int half = (k16 >> 2) & 1;
  const int slot = (k16 & 3) + ((k16 >> 3) << 2);
  return 16 * c2 + 8 * half + slot;
}

template <int DP>
__global__ __launch_bounds__(256) void attention_fwd_kernel(const sf_attention_args a, int vec_qkv,
                                                            int vec_gate) {
  constexpr int KLD = DP + 8;    // K tile row pitch (elements)
  constexpr int VLD = kKT + 8;   // V^T tile row pitch (elements)
  __shared__ __attribute__((aligned(16))) uint16_t sK[kKT * KLD];
  __shared__ __attribute__((aligned(16))) uint16_t sV[DP * VLD];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, li = lane & 31;
  const int bz = blockIdx.z;
  const int b0 = bz / a.B1, b1 = bz - b0 * a.B1;
  const int h = blockIdx.y;
  const int i = blockIdx.x * kQB + wave * 32 + li;
  const bool qin = i < a.Q;
  const int D = a.D, Dv = a.Dv, K = a.K;

  const uint16_t* qp = (const uint16_t*)a.q + b0 * a.q_s[0] + b1 * a.q_s[1] + (int64_t)h * a.q_s[3];
  const uint16_t* kp = (const uint16_t*)a.k + b0 * a.k_s[0] + b1 * a.k_s[1] + (int64_t)h * a.k_s[3];
  const uint16_t* vp = (const uint16_t*)a.v + b0 * a.v_s[0] + b1 * a.v_s[1] + (int64_t)h * a.v_s[3];
  const uint16_t* bp = nullptr;
  if (a.bias)
    bp = (const uint16_t*)a.bias + b0 * a.bias_s[0] + b1 * a.bias_s[1] + (int64_t)h * a.bias_s[2] +
         (int64_t)(qin ? i : 0) * a.bias_s[3];
  const uint8_t* mkp = a.mask_k ? a.mask_k + b0 * a.mk_s[0] + b1 * a.mk_s[1] : nullptr;
  bool qvalid = true;
  if (a.mask_q && qin) qvalid = a.mask_q[b0 * a.mq_s[0] + b1 * a.mq_s[1] + (int64_t)i * a.mq_s[2]] != 0;

  // Q^T as the B operand of S^T = K Q^T: lane holds q[i][16kk + 8*half .. +7].
  bf16x8 qb[DP / 16];
#pragma unroll
  for (int kk = 0; kk < DP / 16; ++kk) {
    u32x4 w = u32x4{0, 0, 0, 0};
    if (qin) w = load8_guard(qp + (int64_t)i * a.q_s[2], 16 * kk + 8 * half, D, vec_qkv);
    qb[kk] = as_bf16x8(w);
  }

  f32x16 o[DP / 32];
#pragma unroll
  for (int db = 0; db < DP / 32; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.f;
  float m = -INFINITY, lsum = 0.f;
  const float c = a.scale * SF_LOG2E;
  const bool use_mask = (a.mask_k != nullptr) || (a.mask_q != nullptr);

  for (int j0 = 0; j0 < K; j0 += kKT) {
    __syncthreads();
    // ---- stage K (row-major) and V^T (slot order) for keys j0 .. j0+63 ----
    for (int t = tid; t < kKT * DP / 8; t += 256) {
      const int r = t / (DP / 8), c8 = (t % (DP / 8)) * 8;
      const int j = j0 + r;
      u32x4 kw = u32x4{0, 0, 0, 0}, vw = u32x4{0, 0, 0, 0};
      if (j < K) {
        kw = load8_guard(kp + (int64_t)j * a.k_s[2], c8, D, vec_qkv);
        vw = load8_guard(vp + (int64_t)j * a.v_s[2], c8, Dv, vec_qkv);
      }
      st16(&sK[r * KLD + c8], kw);
      const int pos = vt_pos(r);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sV[(c8 + 2 * e) * VLD + pos] = (uint16_t)(vw[e] & 0xffff);
        sV[(c8 + 2 * e + 1) * VLD + pos] = (uint16_t)(vw[e] >> 16);
      }
    }
    // key-mask bits for this tile (bit r = key j0 + r valid)
    uint64_t kbits = ~0ull;
    if (use_mask) {
      bool kv = (j0 + lane < K) && (mkp == nullptr || mkp[(int64_t)(j0 + lane) * a.mk_s[2]] != 0);
      kbits = __ballot(kv);
      if (!qvalid) kbits = 0;
    }
    __syncthreads();

    // ---- S^T = K Q^T ----
    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kb][r] = 0.f;
#pragma unroll
      for (int kk = 0; kk < DP / 16; ++kk) {
        bf16x8 ka = as_bf16x8(ld16(&sK[(kb * 32 + li) * KLD + 16 * kk + 8 * half]));
        s[kb] = mfma32(ka, qb[kk], s[kb]);
      }
    }
    // ---- logits in the log2 domain, bias, masks ----
    const uint64_t lbits = kbits >> (4 * half);
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int jl = kb * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        const int j = j0 + jl;
        float t = s[kb][r] * c;
        if (bp != nullptr && j < K) t += bf2f(bp[j]) * SF_LOG2E;
        if (use_mask && !((lbits >> (kb * 32 + 8 * (r >> 2) + (r & 3))) & 1ull)) t = SF_MASKED_LOGIT;
        if (j >= K) t = -INFINITY;
        s[kb][r] = t;
        tmax = fmaxf(tmax, t);
      }
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const float mnew = fmaxf(m, tmax);
    const float alpha = fast_exp2(m - mnew);
    m = mnew;
    lsum *= alpha;
#pragma unroll
    for (int db = 0; db < DP / 32; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[db][r] *= alpha;

    // ---- P = 2^(t - m), O^T += V^T P^T ----
#pragma unroll
    for (int c2 = 0; c2 < 4; ++c2) {
      const int kb = c2 >> 1, base = 8 * (c2 & 1);
      bf16x8 pb;
#pragma unroll
      for (int sl = 0; sl < 8; ++sl) {
        const float p = fast_exp2(s[kb][base + sl] - m);
        lsum += p;
        pb[sl] = (__bf16)p;
      }
#pragma unroll
      for (int db = 0; db < DP / 32; ++db) {
        bf16x8 va = as_bf16x8(ld16(&sV[(db * 32 + li) * VLD + 16 * c2 + 8 * half]));
        o[db] = mfma32(va, pb, o[db]);
      }
    }
  }

  lsum += __shfl_xor(lsum, 32);
  if (!qin) return;
  const float inv = 1.0f / lsum;
  uint16_t* op = (uint16_t*)a.out + b0 * a.o_s[0] + b1 * a.o_s[1] + (int64_t)i * a.o_s[2] +
                 (int64_t)h * a.o_s[3];
  const uint16_t* gp = nullptr;
  if (a.gate)
    gp = (const uint16_t*)a.gate + b0 * a.g_s[0] + b1 * a.g_s[1] + (int64_t)i * a.g_s[2] +
         (int64_t)h * a.g_s[3];
#pragma unroll
  for (int db = 0; db < DP / 32; ++db) {
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
      const int d0 = 32 * db + 8 * c4 + 4 * half;
      if (d0 >= Dv) continue;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = o[db][4 * c4 + e] * inv;
      if (gp != nullptr) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (d0 + e < Dv) v[e] *= sigmoidf_(bf2f(gp[d0 + e]));
      }
      if (vec_gate && d0 + 4 <= Dv) {
        u32x2 w = u32x2{pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3])};
        *reinterpret_cast<u32x2*>(op + d0) = w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (d0 + e < Dv) op[d0 + e] = f2bf(v[e]);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Direct-to-LDS form (16-byte aligned q/k/v rows, head dims multiple of 8, bias rows 8-byte
// aligned).  A wave owns 32 queries of one (batch, head).  Keys stream in tiles of 64:
//   K, V  copied row-major into LDS by global_load_lds_dwordx4 (1 KB per instruction; the
//         16-byte pieces of a K row are XOR-swizzled by key so that the S^T operand reads of
//         consecutive lanes hit distinct banks)
//   S^T   = K Q^T (+ bias tile as the fp32 accumulator seed, + one MFMA k-step that adds the
//         key-mask column: 0, SF_MASKED_LOGIT for masked keys, kPadKey for keys past K)
//   P     = exp(scale (S^T - m)) with the running row maximum m of S^T = q.k + bias / scale
//         (the scale is applied in fp32); lane half h holds keys 8c + 4h + e of each 32-key half
//   O^T  += V^T P^T, the V^T operand read straight from the row-major V tile with
//         ds_read_b64_tr_b16: lane (d, h) of 16-lane group G gets the 4 keys the matching P^T
//         lane holds, for one dim -- no transposed copy of V is ever made.
// SHARED: the 4 waves of a workgroup are consecutive query blocks of one (batch, head) and
// share the K/V tiles (cooperative copy, one barrier per tile).  PRIVATE: every wave is an
// independent (batch, head, query block) task with its own tiles -- for short query ranges
// (atom windows) and for grids too small to fill the GPU with 128-query workgroups.
// ---------------------------------------------------------------------------------------
typedef __attribute__((address_space(3))) uint32_t lds_u32a;
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

constexpr float kPadKey = -8.507059173023462e37f;  // -2^126: keys past K, below any masked key
constexpr float kMassLimit = 1.152921504606846976e18f;   // 2^60: weight mass of a tile that moves m

struct Attn2Plan {
  int QB;            // 32-query blocks per (batch, head)
  // The bias is shared across b0 (samples) and the workgroup count is a multiple of 8: XCD x
  // (workgroup b runs on XCD b % 8) takes the contiguous eighth x of the tasks, ordered b1, head,
  // b0, query block (SHARED) or b1, b0, head, query block (PRIVATE), so that an XCD's L2 holds
  // the bias of the few heads / b1 it serves for all samples, and K/V stay shared between the
  // query blocks (SHARED) or the heads (PRIVATE: neighbouring 64-byte head slices of a K/V row).
  int xcd_order;
  int64_t tasks;     // B0 * B1 * H * QB * ksplit (PRIVATE) or groups of 4 blocks (SHARED)
  int vec_out;       // 8-byte stores of out / loads of gate
  int ksplit;        // PRIVATE: key-range slices per query block (1 = none)
  float* part;       // ksplit > 1: per (block, slice) unnormalised O [32][DP] and (m, l) [32][2]
};

template <int DP>
struct Attn2Tile {
  static constexpr int kRowBytes = DP * 2;
  static constexpr int kKBytes = 64 * kRowBytes;            // one K tile (= one V tile)
  static constexpr int kBufBytes = 2 * kKBytes;             // K + V
  static constexpr int kChunks = kBufBytes / 1024;          // 1 KB copies per tile
  static constexpr int kPieces = DP / 8;                    // 16-byte pieces per row
  static constexpr int kKeysPerChunk = 1024 / kRowBytes;
  __device__ static int kswz(int key) { return DP == 32 ? (key >> 2) & 3 : (key >> 1) & 7; }
  __device__ static int vswz(int key) { return DP == 32 ? 0 : (key >> 1) & 1; }
};

// KC: 16-dim chunks of q.k that hold data (ceil(D / 16)).  BL: the bias tile goes through LDS
// (rows 16-byte aligned, K % 8 == 0): each wave copies its 32 query rows x 64 keys with four
// direct-to-LDS loads of 8 rows x 128 bytes, slot-major [row/8][piece][row%8], and every lane
// then reads its keys with conflict-free 8-byte LDS reads.  Loaded lane by lane from global
// memory instead, every bias instruction touched 32 rows: 40% of the kernel's time.  One buffer
// per wave: the wave reads the tile's bias into registers first, waits for those reads, and only
// then copies the next tile's into the same buffer (48 KB per shared-tile workgroup, three per CU).
template <int DP, bool SHARED, int KC, bool BL>
__global__ __launch_bounds__(256) void attn2_kernel(const sf_attention_args a, const Attn2Plan pl) {
  using T = Attn2Tile<DP>;
  constexpr int kWaveBufs = SHARED ? 1 : 4;                 // tile sets in LDS (shared or per wave)
  constexpr int kKVRegion = kWaveBufs * 2 * T::kBufBytes;
  constexpr int kBiasRegion = BL ? 4 * 4096 : 0;            // per wave: 32 rows x 128 B
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kKVRegion + kBiasRegion];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, li = lane & 31;

  // ---- task of this wave ----
  const int64_t wg = pl.xcd_order ? (int64_t)(blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  int64_t task;
  int qblk;
  if (SHARED) {
    task = wg;                                               // (b, h, group of 4 blocks)
    const int groups = (pl.QB + 3) / 4;
    qblk = (int)(task % groups) * 4 + wave;
    task /= groups;
  } else {
    const int64_t t = wg * 4 + wave;
    if (t >= pl.tasks) return;                               // private waves never meet a barrier
    const int64_t tb = t / pl.ksplit;                        // (batch, head, query block)
    qblk = (int)(tb % pl.QB);
    task = tb / pl.QB;
  }
  // key-range slice of this wave: tiles [t_begin, t_end)
  const int ntiles_all = (a.K + 63) / 64;
  const int slice = SHARED ? 0 : (int)((wg * 4 + wave) % pl.ksplit);
  const int t_begin = (int)((int64_t)ntiles_all * slice / (SHARED ? 1 : pl.ksplit));
  const int t_end = (int)((int64_t)ntiles_all * (slice + 1) / (SHARED ? 1 : pl.ksplit));
  int h, b0, b1;
  if (pl.xcd_order && SHARED) {                              // b1, head, b0
    b0 = (int)(task % a.B0); h = (int)((task / a.B0) % a.H); b1 = (int)(task / ((int64_t)a.B0 * a.H));
  } else if (pl.xcd_order) {                                 // b1, b0, head
    h = (int)(task % a.H); b0 = (int)((task / a.H) % a.B0); b1 = (int)(task / ((int64_t)a.H * a.B0));
  } else {                                                   // b0, b1, head
    h = (int)(task % a.H);
    const int64_t b = task / a.H;
    b0 = (int)(b / a.B1); b1 = (int)(b - (int64_t)b0 * a.B1);
  }
  const int Q = a.Q, K = a.K, D = a.D, Dv = a.Dv;
  const int i = qblk * 32 + li;                              // this lane's query
  const int iq = min(i, Q - 1);
  const bool wactive = qblk * 32 < Q;                        // uniform

  const uint16_t* qp = (const uint16_t*)a.q + b0 * a.q_s[0] + b1 * a.q_s[1] + (int64_t)h * a.q_s[3];
  const char* kp = (const char*)((const uint16_t*)a.k + b0 * a.k_s[0] + b1 * a.k_s[1] + (int64_t)h * a.k_s[3]);
  const char* vp = (const char*)((const uint16_t*)a.v + b0 * a.v_s[0] + b1 * a.v_s[1] + (int64_t)h * a.v_s[3]);
  const uint16_t* bp = a.bias ? (const uint16_t*)a.bias + b0 * a.bias_s[0] + b1 * a.bias_s[1] +
                                    (int64_t)h * a.bias_s[2] + (int64_t)iq * a.bias_s[3]
                              : nullptr;
  const uint8_t* mkp = a.mask_k ? a.mask_k + b0 * a.mk_s[0] + b1 * a.mk_s[1] : nullptr;
  // gathered K / V rows: key j -> row kvip[j] (or the zero row)
  const int32_t* kvip = a.kv_index ? a.kv_index + (int64_t)b1 * a.kvi_s : nullptr;
  const uint8_t* kvmp = a.kv_index && a.kv_mask ? a.kv_mask + (int64_t)b1 * a.kvi_s : nullptr;
  bool qvalid = i < Q;
  if (a.mask_q && i < Q) qvalid = a.mask_q[b0 * a.mq_s[0] + b1 * a.mq_s[1] + (int64_t)i * a.mq_s[2]] != 0;
  const bool any_qmasked = __any(!qvalid && i < Q);          // uniform

  // ---- Q operand (unscaled: S^T holds q.k + bias / scale, scaled in fp32 at the exp) ----
  bf16x8 qb[DP / 16];
#pragma unroll
  for (int kk = 0; kk < DP / 16; ++kk) {
    const int d0 = 16 * kk + 8 * half;
    qb[kk] = as_bf16x8(d0 < D ? ld16(qp + (int64_t)iq * a.q_s[2] + d0) : u32x4{0, 0, 0, 0});
  }
  const float cs = a.scale * SF_LOG2E, inv_scale = 1.0f / a.scale;

  // ---- tile copy: chunk c of a tile, K chunks first ----
  uint8_t* wsm = smem + (SHARED ? 0 : wave * 2 * T::kBufBytes);
  // gathered rows: lane L holds the row of key j0 + L of the next tile to copy (loaded one copy
  // ahead, so that no copy waits for its index)
  int kv_ix = 0, kv_ok = 1;
  auto load_kvrow = [&](int j0) __attribute__((always_inline)) {
    if (kvip != nullptr) {
      const int j = min(j0 + lane, K - 1);
      kv_ix = kvip[j];
      kv_ok = kvmp == nullptr ? 1 : kvmp[j];
    }
  };
  int kv_row = 0;                                            // kv_ix / kv_ok resolved for the copy
  auto copy_chunk = [&](int c, int j0, int buf) __attribute__((always_inline)) {
    const bool isk = c < T::kChunks / 2;
    const int cc = isk ? c : c - T::kChunks / 2;
    const int key = cc * T::kKeysPerChunk + lane / T::kPieces;
    const int slot = lane % T::kPieces;
    int piece = slot ^ (isk ? T::kswz(key) : T::vswz(key));
    if (8 * piece >= (isk ? D : Dv)) piece = 0;              // dims past D: any finite data
    int row = min(j0 + key, K - 1);
    if (kvip != nullptr) row = __shfl(kv_row, key);
    const char* src = (isk ? kp + (int64_t)row * a.k_s[2] * 2 : vp + (int64_t)row * a.v_s[2] * 2) + piece * 16;
    __builtin_amdgcn_global_load_lds(src, (lds_u32a*)(wsm + buf * T::kBufBytes + c * 1024), 16, 0, 0);
  };
  auto copy_tile = [&](int j0, int buf) __attribute__((always_inline)) {
    if (kvip != nullptr) {
      kv_row = kv_ok == 0 || kv_ix < 0 || kv_ix >= a.kv_zero_row ? a.kv_zero_row : kv_ix;
      load_kvrow(j0 + 64);                                   // the next copy's rows
    }
    if (SHARED) {
#pragma unroll
      for (int u = 0; u < T::kChunks / 4; ++u) copy_chunk(wave * (T::kChunks / 4) + u, j0, buf);
    } else {
#pragma unroll
      for (int u = 0; u < T::kChunks; ++u) copy_chunk(u, j0, buf);
    }
  };
  // ---- bias tile (this lane's query, its 32 keys) and key-mask bits ----
  u32x2 bnext[8];
  // key-mask byte of key j0 + lane of the next tile, kept raw until the tile's wait: a ballot
  // right after the load waited for it -- and, the vector memory counter being in order, for the
  // next tile's copies issued just before, which serialised the prefetch with the compute
  // (diffusion 5 x 1024: 0.155 -> 0.140 ms per block)
  uint32_t mbyte = 1;
  uint8_t* bsm = smem + kKVRegion + wave * 4096;            // BL: this wave's bias buffer
  // BL source rows: lane L copies row 8u + L/8 of the wave's 32 queries, piece (L%8) ^ (L/8)
  // (keys 8p .. 8p+7): the 8 lanes of a row read its 128 bytes, so every 4 consecutive lanes read
  // 64 contiguous bytes (with a query row per lane, consecutive lanes on different rows, the same
  // copies ran at a third of the L2 bandwidth), and the XOR spreads a column of pieces over the
  // LDS banks for the reads below.
  const int bpiece = (lane & 7) ^ (lane >> 3);
  const uint16_t* brow0 = nullptr;
  int64_t brs8 = 0;                                          // elements between rows 8 apart
  if (BL) {
    const uint16_t* bh = (const uint16_t*)a.bias + b0 * a.bias_s[0] + b1 * a.bias_s[1] + (int64_t)h * a.bias_s[2];
    brow0 = bh + (int64_t)min(qblk * 32 + (lane >> 3), Q - 1) * a.bias_s[3] + 8 * bpiece;
    brs8 = 8 * a.bias_s[3];
  }
  const bool brows_clamped = qblk * 32 + 32 > Q;            // uniform: the last query block
  auto load_bias_lds = [&](int j0) __attribute__((always_inline)) {
    const int jc = min(j0, K - 8 - 8 * bpiece) - j0;         // pieces past K re-read the last one
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint16_t* src = brow0 + u * brs8;
      if (brows_clamped) {
        const uint16_t* bh = (const uint16_t*)a.bias + b0 * a.bias_s[0] + b1 * a.bias_s[1] + (int64_t)h * a.bias_s[2];
        src = bh + (int64_t)min(qblk * 32 + 8 * u + (lane >> 3), Q - 1) * a.bias_s[3] + 8 * bpiece;
      }
      __builtin_amdgcn_global_load_lds(src + j0 + jc, (lds_u32a*)(bsm + u * 1024), 16, 0, 0);
    }
  };
  auto load_side = [&](int j0) __attribute__((always_inline)) {
    if (BL) {
    } else if (bp == nullptr) {
#pragma unroll
      for (int q = 0; q < 8; ++q) bnext[q] = u32x2{0, 0};
    } else if (j0 + 64 <= K) {                               // uniform: the whole tile is in range
#pragma unroll
      for (int q = 0; q < 8; ++q)                            // keys j0 + 32(q/4) + 8(q%4) + 4half .. +3
        bnext[q] = *reinterpret_cast<const u32x2*>(bp + j0 + 32 * (q >> 2) + 8 * (q & 3) + 4 * half);
    } else {                                                 // last tile: ragged end of the keys
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int j = j0 + 32 * (q >> 2) + 8 * (q & 3) + 4 * half;
        uint16_t t[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) t[e] = j + e < K ? bp[j + e] : 0;
        bnext[q] = u32x2{(uint32_t)t[0] | ((uint32_t)t[1] << 16), (uint32_t)t[2] | ((uint32_t)t[3] << 16)};
      }
    }
    if (mkp != nullptr) mbyte = mkp[(int64_t)min(j0 + lane, K - 1) * a.mk_s[2]];
  };
  // valid keys of the tile at j0, once its mask bytes (load_side(j0)) have landed
  auto mask_bits = [&](int j0) __attribute__((always_inline)) -> uint64_t {
    return __ballot(j0 + lane < K && mbyte != 0);
  };

  f32x16 o[DP / 32];
#pragma unroll
  for (int db = 0; db < DP / 32; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.f;
  float m = -INFINITY, l = 0.f;
  bf16x8 ones_b;                                             // B operand: 1 at k = 0 (half 0)
#pragma unroll
  for (int e = 0; e < 8; ++e) ones_b[e] = (__bf16)((e == 0 && half == 0) ? 1.0f : 0.0f);

  // Waits: the copies into LDS are ordinary loads to the compiler, so every wait is followed
  // by a compiler barrier (or __syncthreads) that keeps the LDS reads of the tile after it.
  load_kvrow(t_begin * 64);
  copy_tile(t_begin * 64, 0);
  if (BL) load_bias_lds(t_begin * 64);
  load_side(t_begin * 64);
  __builtin_amdgcn_s_waitcnt(0);
  if (SHARED) __syncthreads();
  else asm volatile("" ::: "memory");

  for (int t = t_begin; t < t_end; ++t) {
    const int buf = (t - t_begin) & 1, j0 = t * 64;
    const uint8_t* kt = wsm + buf * T::kBufBytes;
    const uint8_t* vt = kt + T::kKBytes;
    u32x2 bcur[8];
    if (BL) {                                                // keys 32(q/4) + 8(q%4) + 4half .. +3 = piece q
#pragma unroll
      for (int q = 0; q < 8; ++q)                            // row li: slot 8 (li%8) + (q ^ li%8) of chunk li/8
        bcur[q] = *reinterpret_cast<const u32x2*>(bsm + (li >> 3) * 1024 + (li & 7) * 128 + (q ^ (li & 7)) * 16 + half * 8);
      // the buffer is refilled below: these reads complete first (the copies are ordinary loads
      // to the compiler, so the wait carries a memory clobber)
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q) bcur[q] = bnext[q];
    }
    const uint64_t mbits = mask_bits(j0);
    if (t + 1 < t_end) {
      copy_tile(j0 + 64, buf ^ 1);
      if (BL) load_bias_lds(j0 + 64);
      load_side(j0 + 64);
    }
    if (wactive) {
      // ---- S^T = K Q^T + bias (+ mask column) ----
      const bool need_mask = mbits != ~0ull;                 // uniform
      f32x16 s[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            s[kb][4 * c + 2 * e] = bflo(bcur[4 * kb + c][e]) * inv_scale;
            s[kb][4 * c + 2 * e + 1] = bfhi(bcur[4 * kb + c][e]) * inv_scale;
          }
        const int key = 32 * kb + li;
#pragma unroll
        for (int kk = 0; kk < KC; ++kk) {                    // chunks past D are zeros in q
          const int piece = (2 * kk + half) ^ T::kswz(key);
          s[kb] = mfma32(as_bf16x8(ld16(kt + key * T::kRowBytes + piece * 16)), qb[kk], s[kb]);
        }
        if (need_mask) {
          bf16x8 mc;
#pragma unroll
          for (int e = 0; e < 8; ++e) mc[e] = (__bf16)0.0f;
          const float mv = ((mbits >> key) & 1ull) ? 0.0f : (j0 + key < K ? SF_MASKED_LOGIT : kPadKey);
          mc[0] = (__bf16)(half == 0 ? mv : 0.0f);
          s[kb] = mfma32(mc, ones_b, s[kb]);
        }
      }
      if (any_qmasked && !qvalid) {                          // masked query: uniform over keys < K
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            s[kb][r] = j0 + 32 * kb + 8 * (r >> 2) + 4 * half + (r & 3) < K ? 0.0f : kPadKey;
      }
      // ---- softmax against a reference point m (in units of S^T) ----
      // Tile 0 sets m to the row maximum of its 64 keys.  Later tiles keep it unless the
      // probability mass of the tile exceeds kMassLimit (all weights are >= 0, so the sum bounds
      // every weight and an overflow cannot pass unnoticed); then m moves to the tile's maximum
      // and what is accumulated is rescaled.  This replaces a running maximum (a max over the
      // tile, one exp and a rescale of O every tile) by one compare.
      auto row_max = [&]() __attribute__((always_inline)) {
        float v = s[0][0];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) v = fmaxf(v, s[kb][r]);
        return fmaxf(v, __shfl_xor(v, 32));
      };
      auto weights = [&](float mref, bf16x2 (&pw)[16]) __attribute__((always_inline)) {
        const float mb = mref * cs;
        float t0 = 0.f, t1 = 0.f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            pw[8 * kb + e] = cvt_bf2(fast_exp2(__builtin_fmaf(s[kb][2 * e], cs, -mb)),
                                     fast_exp2(__builtin_fmaf(s[kb][2 * e + 1], cs, -mb)));
            if (e & 1) t1 = add_bf2(pw[8 * kb + e], t1); else t0 = add_bf2(pw[8 * kb + e], t0);
          }
        return t0 + t1;
      };
      if (t == t_begin) m = row_max();
      bf16x2 pw[16];
      float ts = weights(m, pw);
      if (__any(!(ts <= kMassLimit))) {                      // rare: move m up and rescale
        const float mnew = fmaxf(m, row_max());
        const float alpha = fast_exp2((m - mnew) * cs);
        m = mnew;
        l *= alpha;
#pragma unroll
        for (int db = 0; db < DP / 32; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
        ts = weights(m, pw);
      }
      l += ts;
      // ---- O^T += V^T P^T ----
      const int grp = lane >> 4, gi = lane & 15;            // 16-lane group, index in group
      const int ekey = gi >> 2, q4 = gi & 3;                 // source lane: key e, dims 4q .. 4q+3
#pragma unroll
      for (int c2 = 0; c2 < 4; ++c2) {
        bf16x8 pb;
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2) {
          pb[2 * q2] = pw[4 * c2 + q2][0];
          pb[2 * q2 + 1] = pw[4 * c2 + q2][1];
        }
#pragma unroll
        for (int db = 0; db < DP / 32; ++db) {
          const int d = 32 * db + 16 * (grp & 1) + 4 * q4;
          u32x2 part[2];                // moved as 32-bit words: no 16-bit element extraction
#pragma unroll
          for (int rd = 0; rd < 2; ++rd) {
            const int key = 16 * c2 + 8 * rd + 4 * (grp >> 1) + ekey;
            const int off = key * T::kRowBytes + (((d >> 3) ^ T::vswz(key)) << 4) + ((d >> 2) & 1) * 8;
            part[rd] = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(vt + off)));
          }
          const bf16x8 va = as_bf16x8(u32x4{part[0][0], part[0][1], part[1][0], part[1][1]});
          o[db] = mfma32(va, pb, o[db]);
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0);                           // next tile, bias and mask landed
    if (SHARED) __syncthreads();
    else asm volatile("" ::: "memory");
  }

  // ---- epilogue: O / l, optional sigmoid gate ----
  if (!wactive || i >= Q) return;
  const float lt = l + __shfl_xor(l, 32);
  if (!SHARED && pl.ksplit > 1) {
    // one slice of the keys: unnormalised O, its reference point and weight sum, for the combine
    const int64_t slot = wg * 4 + wave;                      // (block, slice) in task order
    float* po = pl.part + slot * 32 * (DP + 2);
#pragma unroll
    for (int db = 0; db < DP / 32; ++db)
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4)
        *reinterpret_cast<f32x4*>(po + li * DP + 32 * db + 8 * c4 + 4 * half) =
            f32x4{o[db][4 * c4], o[db][4 * c4 + 1], o[db][4 * c4 + 2], o[db][4 * c4 + 3]};
    if (half == 0) *reinterpret_cast<f32x2*>(po + 32 * DP + 2 * li) = f32x2{m, lt};
    return;
  }
  const float inv = 1.0f / lt;
  uint16_t* op = (uint16_t*)a.out + b0 * a.o_s[0] + b1 * a.o_s[1] + (int64_t)i * a.o_s[2] + (int64_t)h * a.o_s[3];
  const uint16_t* gp = a.gate ? (const uint16_t*)a.gate + b0 * a.g_s[0] + b1 * a.g_s[1] + (int64_t)i * a.g_s[2] +
                                    (int64_t)h * a.g_s[3]
                              : nullptr;
#pragma unroll
  for (int db = 0; db < DP / 32; ++db) {
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
      const int d0 = 32 * db + 8 * c4 + 4 * half;
      if (d0 >= Dv) continue;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = o[db][4 * c4 + e] * inv;
      const bool full = d0 + 4 <= Dv && pl.vec_out;
      if (gp != nullptr) {
        if (full) {
          const u32x2 gw = *reinterpret_cast<const u32x2*>(gp + d0);
          v[0] *= sigmoidf_(bflo(gw[0])); v[1] *= sigmoidf_(bfhi(gw[0]));
          v[2] *= sigmoidf_(bflo(gw[1])); v[3] *= sigmoidf_(bfhi(gw[1]));
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (d0 + e < Dv) v[e] *= sigmoidf_(bf2f(gp[d0 + e]));
        }
      }
      if (full) {
        *reinterpret_cast<u32x2*>(op + d0) = u32x2{pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3])};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (d0 + e < Dv) op[d0 + e] = f2bf(v[e]);
      }
    }
  }
}

// Combine of the key-range slices: thread per (query block, query, 4 dims).  O and l of each
// slice are relative to the slice's own reference point m_s; with M = max m_s the result is
// sum_s O_s 2^(cs (m_s - M)) / sum_s l_s 2^(cs (m_s - M)), then the gate.  All loads of a thread
// are independent and issued together: one memory round trip per thread.
template <int DP, int KS>
__global__ __launch_bounds__(256) void attn2_combine_kernel(const sf_attention_args a, const Attn2Plan pl) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t nblk = pl.tasks / KS;
  if (t >= nblk * 32 * (DP / 4)) return;
  const int d0 = 4 * (int)(t % (DP / 4));
  const int li = (int)((t / (DP / 4)) % 32);
  const int64_t blk = t / (32 * (DP / 4));                  // a PRIVATE task in the kernel's order
  const int qblk = (int)(blk % pl.QB);
  const int64_t task = blk / pl.QB;
  int h, b0, b1;
  if (pl.xcd_order) {                                        // b1, b0, head
    h = (int)(task % a.H); b0 = (int)((task / a.H) % a.B0); b1 = (int)(task / ((int64_t)a.H * a.B0));
  } else {
    h = (int)(task % a.H);
    const int64_t b = task / a.H;
    b0 = (int)(b / a.B1); b1 = (int)(b - (int64_t)b0 * a.B1);
  }
  const int i = qblk * 32 + li;
  if (i >= a.Q || d0 >= a.Dv) return;
  const float cs = a.scale * SF_LOG2E;
  const float* base = pl.part + blk * KS * 32 * (DP + 2);
  f32x2 ml[KS];
  f32x4 os[KS];
#pragma unroll
  for (int sl = 0; sl < KS; ++sl) {
    ml[sl] = *reinterpret_cast<const f32x2*>(base + sl * 32 * (DP + 2) + 32 * DP + 2 * li);
    os[sl] = *reinterpret_cast<const f32x4*>(base + sl * 32 * (DP + 2) + li * DP + d0);
  }
  float mx = ml[0][0];
#pragma unroll
  for (int sl = 1; sl < KS; ++sl) mx = fmaxf(mx, ml[sl][0]);
  float lsum = 0.f, v[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int sl = 0; sl < KS; ++sl) {
    const float w = fast_exp2((ml[sl][0] - mx) * cs);
    lsum += w * ml[sl][1];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] += w * os[sl][e];
  }
  const float inv = 1.0f / lsum;
  uint16_t* op = (uint16_t*)a.out + b0 * a.o_s[0] + b1 * a.o_s[1] + (int64_t)i * a.o_s[2] + (int64_t)h * a.o_s[3];
  const uint16_t* gp = a.gate ? (const uint16_t*)a.gate + b0 * a.g_s[0] + b1 * a.g_s[1] + (int64_t)i * a.g_s[2] +
                                    (int64_t)h * a.g_s[3]
                              : nullptr;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (d0 + e >= a.Dv) continue;
    float x = v[e] * inv;
    if (gp != nullptr) x *= sigmoidf_(bf2f(gp[d0 + e]));
    op[d0 + e] = f2bf(x);
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7) == 0; }

}  // namespace

namespace {

struct AttnRoute {
  bool vec, vec_out, attn2, shared, bl;
  int dmax, kc, ksplit;
  Attn2Plan pl;
};

int route(const sf_attention_args* a, bool allow_split, AttnRoute& r) {
  if (a->q == nullptr || a->k == nullptr || a->v == nullptr || a->out == nullptr) {
    sf_set_error("attention: q, k, v and out must be non-null"); return 1;
  }
  if (a->B0 <= 0 || a->B1 <= 0 || a->Q <= 0 || a->K <= 0 || a->H <= 0 || a->D <= 0 || a->Dv <= 0) {
    sf_set_error("attention: sizes must be positive (B0=%d B1=%d Q=%d K=%d H=%d D=%d Dv=%d)",
                 a->B0, a->B1, a->Q, a->K, a->H, a->D, a->Dv);
    return 1;
  }
  r.dmax = a->D > a->Dv ? a->D : a->Dv;
  if (r.dmax > 64) { sf_set_error("attention: head dims above 64 are not supported (D=%d Dv=%d)", a->D, a->Dv); return 1; }
  if ((int64_t)a->B0 * a->B1 > 65535 || a->H > 65535) {
    sf_set_error("attention: batch (%d) or heads (%d) exceed the grid limit", a->B0 * a->B1, a->H); return 1;
  }
  // 16-byte path for q/k/v rows: head dims multiple of 8, row/head strides multiple of 8,
  // 16-byte aligned bases.
  r.vec = (a->D % 8 == 0) && (a->Dv % 8 == 0) && aligned16(a->q) && aligned16(a->k) && aligned16(a->v);
  for (int s = 0; s < 4 && r.vec; ++s)
    r.vec = (a->q_s[s] % 8 == 0) && (a->k_s[s] % 8 == 0) && (a->v_s[s] % 8 == 0);
  r.vec_out = aligned8(a->out);
  for (int s = 0; s < 4 && r.vec_out; ++s) r.vec_out = (a->o_s[s] % 4 == 0);
  bool bias_vec = a->bias == nullptr || aligned8(a->bias);
  for (int s = 0; s < 4 && bias_vec && a->bias != nullptr; ++s) bias_vec = a->bias_s[s] % 4 == 0;
  r.attn2 = r.vec && bias_vec;
  r.ksplit = 1;
  r.pl = Attn2Plan{};
  if (a->kv_index != nullptr && (!r.attn2 || a->kv_zero_row < 0)) {
    sf_set_error("attention: gathered K/V rows need 16-byte aligned q/k/v rows and strides, an 8-byte aligned "
                 "bias and kv_zero_row >= 0");
    return 1;
  }
  if (!r.attn2) return 0;
  Attn2Plan& pl = r.pl;
  pl.QB = (a->Q + 31) / 32;
  pl.vec_out = r.vec_out && (a->gate == nullptr || aligned8(a->gate));
  for (int s = 0; s < 4 && pl.vec_out && a->gate != nullptr; ++s) pl.vec_out = a->g_s[s] % 4 == 0;
  const int64_t bh = (int64_t)a->B0 * a->B1 * a->H;
  const int64_t groups = bh * ((pl.QB + 3) / 4);
  r.shared = a->schedule == 0 ? (a->Q >= 128 && groups >= 512) : a->schedule == 1;
  // Per-wave tasks on a grid too small for the GPU (single attention: 16 heads x 24 blocks =
  // 384 waves for 1024 SIMDs) split their key range into slices of >= 2 tiles, up to ~2048 waves;
  // a combine kernel merges the slices.  Needs a workspace (module-level entry points).
  if (allow_split && !r.shared) {
    const int ntiles = (a->K + 63) / 64;
    const int64_t blocks = bh * pl.QB;
    int ks = (int)((2048 + blocks - 1) / blocks);
    ks = ks < 4 ? ks : 4;
    ks = ks < ntiles / 2 ? ks : ntiles / 2;
    r.ksplit = ks > 1 ? ks : 1;
  }
  pl.ksplit = r.ksplit;
  pl.tasks = r.shared ? groups : bh * pl.QB * r.ksplit;
  const int64_t wgs = r.shared ? pl.tasks : (pl.tasks + 3) / 4;
  pl.xcd_order = a->bias != nullptr && a->bias_s[0] == 0 && a->B0 > 1 && wgs % 8 == 0 && (r.shared || pl.tasks % 4 == 0);
  r.kc = (a->D + 15) / 16;                                  // q.k chunks holding data
  // LDS bias tiles: always with shared tiles; per-wave tiles from two key tiles on (with one
  // bias buffer per wave a per-wave-tile workgroup takes 80 KB, two per CU as without the bias
  // tiles: atom windows, K = 128, 34.7 -> 30.5 us; single attention, K = 768, 30 -> 25 us)
  r.bl = a->bias != nullptr && aligned16(a->bias) && a->K % 8 == 0 && (r.shared || a->K >= 128);
  for (int s2 = 0; s2 < 4 && r.bl; ++s2) r.bl = a->bias_s[s2] % 8 == 0;
  return 0;
}

size_t split_bytes(const sf_attention_args* a, const AttnRoute& r) {
  if (!r.attn2 || r.ksplit <= 1) return 0;
  const int dp = r.dmax <= 32 ? 32 : 64;
  return (size_t)r.pl.tasks * 32 * (dp + 2) * sizeof(float);
}

int launch_attention(const sf_attention_args* a, const AttnRoute& r, float* split_ws, hipStream_t st) {
  if (r.attn2) {
    Attn2Plan pl = r.pl;
    pl.part = split_ws;
    const int64_t wgs = r.shared ? pl.tasks : (pl.tasks + 3) / 4;
    if (wgs > 0x7fffffff) { sf_set_error("attention: problem too large for the grid"); return 1; }
    const dim3 g2((unsigned)wgs);
    auto launch = [&](auto dp, auto sh, auto kcc, auto blc) {
      hipLaunchKernelGGL((attn2_kernel<decltype(dp)::value, decltype(sh)::value, decltype(kcc)::value,
                                       decltype(blc)::value>), g2, dim3(256), 0, st, *a, pl);
    };
    using I32 = std::integral_constant<int, 32>;
    using I64 = std::integral_constant<int, 64>;
    using Tt = std::true_type;
    using Ff = std::false_type;
    auto by_bl = [&](auto dp, auto sh, auto kcc) {
      if (r.bl) launch(dp, sh, kcc, Tt{});
      else launch(dp, sh, kcc, Ff{});
    };
    auto by_sh = [&](auto dp, auto kcc) {
      if (r.shared) by_bl(dp, Tt{}, kcc);
      else by_bl(dp, Ff{}, kcc);
    };
    if (r.dmax <= 32) {
      if (r.kc <= 1) by_sh(I32{}, std::integral_constant<int, 1>{});
      else by_sh(I32{}, std::integral_constant<int, 2>{});
    } else if (r.kc <= 3) {
      by_sh(I64{}, std::integral_constant<int, 3>{});
    } else {
      by_sh(I64{}, std::integral_constant<int, 4>{});
    }
    int rc = sf_check_launch("attn2_kernel");
    if (rc || pl.ksplit <= 1) return rc;
    const int dp = r.dmax <= 32 ? 32 : 64;
    const int64_t threads = pl.tasks / pl.ksplit * 32 * (dp / 4);
    const dim3 gc((unsigned)((threads + 255) / 256));
    auto combine = [&](auto ks) {
      constexpr int KS = decltype(ks)::value;
      if (dp == 32) hipLaunchKernelGGL((attn2_combine_kernel<32, KS>), gc, dim3(256), 0, st, *a, pl);
      else hipLaunchKernelGGL((attn2_combine_kernel<64, KS>), gc, dim3(256), 0, st, *a, pl);
    };
    if (pl.ksplit > 8) { sf_set_error("attention: at most 8 key-range slices"); return 1; }
    switch (pl.ksplit) {
      case 2: combine(std::integral_constant<int, 2>{}); break;
      case 3: combine(std::integral_constant<int, 3>{}); break;
      case 4: combine(std::integral_constant<int, 4>{}); break;
      case 5: combine(std::integral_constant<int, 5>{}); break;
      case 6: combine(std::integral_constant<int, 6>{}); break;
      case 7: combine(std::integral_constant<int, 7>{}); break;
      default: combine(std::integral_constant<int, 8>{}); break;
    }
    return sf_check_launch("attn2_combine_kernel");
  }
  dim3 grid((a->Q + kQB - 1) / kQB, a->H, a->B0 * a->B1);
  if (r.dmax <= 32)
    hipLaunchKernelGGL(attention_fwd_kernel<32>, grid, dim3(256), 0, st, *a, (int)r.vec, (int)r.vec_out);
  else
    hipLaunchKernelGGL(attention_fwd_kernel<64>, grid, dim3(256), 0, st, *a, (int)r.vec, (int)r.vec_out);
  return sf_check_launch("attention_fwd_kernel");
}

}  // namespace

size_t sf_attention_workspace_bytes(const sf_attention_args* a) {
  AttnRoute r;
  if (a == nullptr || route(a, true, r)) return 0;
  return split_bytes(a, r);
}

int sf_attention_run(const sf_attention_args* a, void* workspace, size_t workspace_bytes, hipStream_t st) {
  if (a == nullptr) { sf_set_error("attention: null args"); return 1; }
  if (a->schedule == 3) {
    // the shared-bias kernel, opt-in: on the diffusion shape it measured slower than the
    // shared-tile kernel (51.5 against 45 us), so the automatic choice never takes it
    const char* why = nullptr;
    AttnRoute chk;
    if (route(a, false, chk)) return 1;                      // argument checks first
    if (sf_sb_attention_ok(a, &why)) return sf_sb_attention_launch(a, st);
    sf_set_error("attention: schedule 3 (shared-bias kernel) refused: %s", why);
    return 1;
  }
  AttnRoute r;
  const bool can_split = workspace != nullptr;
  if (route(a, can_split, r)) return 1;
  if (can_split && split_bytes(a, r) > workspace_bytes) {
    // the caller sized its workspace for a different route: run without slices
    if (route(a, false, r)) return 1;
  }
  return launch_attention(a, r, static_cast<float*>(workspace), st);
}

extern "C" int sf_hip_attention_fwd(const sf_attention_args* a, void* stream) {
  return sf_attention_run(a, nullptr, 0, reinterpret_cast<hipStream_t>(stream));
}
