// Gated pair-biased attention whose bias is shared by every sample of the batch, for head
// dim 48: the diffusion transformer's token attention (5 samples of one example attend with
// the same [H, N, N] pair bias; DiffusionSelfAttention.cpp:391,555 index the bias with
// batch % pair_batch_count, transformer.py:306-345 the module).
//
// Work decomposition: one workgroup = 4 waves = (head h, 64 queries); wave w takes 32 of the
// queries (w & 1) for ALL samples of the batch and one half of the keys (w >> 1), one wave per
// SIMD.  Per 32-key tile the wave loads its 32 x 32 bias block once, straight into registers,
// and serves every sample from it:
//   seed   = bias^T * log2 e in S^T register order, from two identity MFMAs on the 16-byte
//            bias loads (the keys of a lane's load are contiguous; the identity places them)
//   S^T_s  = K_s Q_s'^T + seed       3 x 32x32x16 MFMAs (48 dims, no padding on q.k)
//   P_s    = 2^S (fixed reference point 0: Q' carries scale * log2 e)
//   O_s^T += V_s^T P_s^T             dims 0-31: 2 MFMAs; dims 32-47 plus the row sum: 2 MFMAs
//            whose A operand rows 16-31 are the constant rows of the V tile (row 16 all ones,
//            the rest zeros), so that O^T row 48 is the weight sum l -- a 16-wide MFMA for the
//            last 16 dims and a separate row-sum MFMA would take the same matrix-core time
// K and V tiles of all samples for both key halves are double-buffered in LDS by
// direct-to-LDS buffer loads.  At the end the two key halves of a query block add their O
// and l through LDS (same reference point: a plain sum), each wave finishing the samples it
// owns: O / l, the sigmoid gate, bf16 stores.
//
// The fixed reference point needs no running maximum, no rescale and no per-score subtract
// (the exponentials are the VALU's largest cost).  A (sample, query) whose weight sum leaves
// [2^-100, 2^100] (an overflow, an underflow of the whole row, or every key masked) is
// recomputed by the owning wave with an exact two-pass softmax from global memory; a query
// whose keys are all masked gets the mean of V over all keys (the reference's -finfo.max
// additive mask, sdpa.py:62-80).
//
// The 5 samples' O accumulators (160 registers per lane) live in AGPRs, written only by the P.V
// MFMAs (inline assembly with AGPR operands); every other MFMA accumulates in VGPRs.  One wave
// per SIMD (236 VGPRs, 160 AGPRs), so the P.V MFMAs run one sample behind the exponentials to
// keep the in-order issue from stalling on dependent MFMAs, and the next tile's copies are
// issued over the first three sample steps.  The LDS operand reads and the bias loads are
// inline assembly with explicit waits; each such load's destination stays live (used after the
// wait that covers it), which is what makes the asynchronous write safe.
//
// Measured on the diffusion shape (5 x 1024 tokens, 16 heads): 51.5 us against 45 us for the
// shared-tile kernel (attn2_kernel), so it is opt-in (schedule 3).  Per 32-key tile a wave
// spends ~1000 cycles of its ~4900 issuing its 17-18 direct-to-LDS copies (each waits ~70
// cycles for the texture unit, shared by the four waves of the CU) and ~900 waiting for the
// copies and the barrier; with one wave per SIMD nothing hides those stalls.
#include "sf_common.h"

namespace {

constexpr int kSbR = 5;                      // samples per wave
constexpr int kSbD = 48;                     // head dim
constexpr int kSbKT = 32;                    // keys per tile
constexpr int kSbKRow = kSbD * 2;            // K row in LDS: 96 bytes (6 pieces of 16)
constexpr int kSbVRow = 128;                 // V row in LDS: 6 data pieces + 2 constant pieces
constexpr int kSbKTile = kSbKT * kSbKRow;    // 3072
constexpr int kSbVTile = kSbKT * kSbVRow;    // 4096
constexpr int kSbPair = kSbKTile + kSbVTile; // one (key half, sample): K tile then V tile
constexpr int kSbStage = 2 * kSbR * kSbPair; // 71680
constexpr int kSbMaskOff = 2 * kSbStage;     // key-mask bit words
constexpr int kSbMaxK = 4096;
constexpr int kSbLds = kSbMaskOff + kSbMaxK / 8;
constexpr int kSbPartRegs = 25;              // O^T registers per lane that hold data (16 + 8 + l)
static_assert(kSbR * kSbPartRegs * 2 * 256 <= 2 * kSbStage, "partials fit the tile buffers");

typedef __attribute__((address_space(3))) uint32_t lds_u32s;
typedef short sb_v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) sb_v4i16 lds_v4i16s;

constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit data (gfx9 family)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t sb_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, (int)kRsrcWord3);
}

// ds_read_b64_tr_b16 as inline assembly: with the builtin the compiler waits for every
// outstanding direct-to-LDS copy (the next tile's included) before each read.  The caller
// waits (lgkmcnt) before using the result.
template <int OFF = 0>
__device__ __forceinline__ u32x2 tr_read_off(uint32_t addr) {
  u32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}

// O^T += V^T P^T for one dim block, as inline assembly so that the accumulators stay in AGPRs
// (every other MFMA of the kernel accumulates in VGPRs).  NOPS wait states first when the P^T
// operand was just written by the VALU; back-to-back MFMAs on one accumulator need none.
template <int NOPS>
__device__ __forceinline__ void pv1(f32x16& o, const u32x4& va, const bf16x8& pb) {
  if constexpr (NOPS > 0)
    asm volatile("s_nop %3\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(o) : "v"(va), "v"(pb), "i"(NOPS));
  else
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(o) : "v"(va), "v"(pb));
}

template <int OFF>
__device__ __forceinline__ u32x4 ds_read16_off(uint32_t addr) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}

struct SbArgs {
  sf_attention_args a;
  uint32_t qkv_bytes;       // buffer extents (bytes from each head's base)
  uint32_t bias_bytes;
  int xcd;                  // task order XCD-contiguous (grid a multiple of 8)
};

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void sb_attn_kernel(const SbArgs args) {
  const sf_attention_args& a = args.a;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kSbLds];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kh = wave >> 1, qs = wave & 1;
  const int hf = lane >> 5, li = lane & 31;
  const int grp = lane >> 4, gi = lane & 15;

  const int QB = a.Q / 64;
  const int tasks = QB * a.H;
  int task = blockIdx.x;
  if (args.xcd) task = (blockIdx.x & 7) * (tasks >> 3) + (blockIdx.x >> 3);
  const int h = task / QB, qb = task - h * QB;
  const int q0 = qb * 64 + qs * 32;             // this wave's first query
  const int K = a.K, nt = K / 64;               // tiles per key half
  const int kbeg = kh * (K / 2);

  // ---- buffer resources: K, V, bias of head h (sample and tile offsets go to soffset) ----
  const uint16_t* kbase = (const uint16_t*)a.k + (int64_t)h * a.k_s[3];
  const uint16_t* vbase = (const uint16_t*)a.v + (int64_t)h * a.v_s[3];
  const uint16_t* bbase = (const uint16_t*)a.bias + (int64_t)h * a.bias_s[2];
  const __amdgpu_buffer_rsrc_t rk = sb_rsrc(kbase, args.qkv_bytes);
  const __amdgpu_buffer_rsrc_t rv = sb_rsrc(vbase, args.qkv_bytes);
  const uint32_t krs = (uint32_t)a.k_s[2] * 2, vrs = (uint32_t)a.v_s[2] * 2;   // row strides (bytes)
  const uint32_t kss = (uint32_t)a.k_s[0] * 2, vss = (uint32_t)a.v_s[0] * 2;   // sample strides

  // ---- tile copies: the two waves of a key half split its K and V tiles, wave (kh, qs) taking
  //      the K tile of samples s with s + qs even and the V tile of the others (17 and 18 copies).
  //      K: slot 64u + L -> key slot / 6, position slot % 6 holding piece position ^ ((key >> 3)
  //      & 1) (the S^T operand reads are then conflict-free).  V: slot 64u + L -> key slot / 8,
  //      position slot % 8 holding piece position ^ (key & 2) << 1; pieces 6 and 7 are the
  //      constant rows (never copied: those lanes sit out). ----
  uint32_t kcofs[3], vcofs[4];
  bool vlane = true;                                     // V: this lane's slots hold data pieces
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int slot = 64 * u + lane;
    if (u < 3) {
      const int key = slot / 6, pos = slot - 6 * (slot / 6);
      kcofs[u] = (uint32_t)key * krs + 16u * (pos ^ ((key >> 3) & 1));
    }
    const int vkey_ = slot >> 3, piece = (slot & 7) ^ ((vkey_ & 2) << 1);   // the same for every u
    vcofs[u] = (uint32_t)vkey_ * vrs + 16u * (piece < 6 ? piece : 0);
    vlane = piece < 6;
  }
  auto copy_sample = [&](int t, int stage, int s) __attribute__((always_inline)) {
    const uint32_t j0 = (uint32_t)(kbeg + t * kSbKT);
    uint8_t* dst = smem + stage * kSbStage + (kh * kSbR + s) * kSbPair;
    if (((s + qs) & 1) == 0) {
      const uint32_t so = (uint32_t)s * kss + j0 * krs;
#pragma unroll
      for (int u = 0; u < 3; ++u)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_u32s*)(dst + 1024 * u), 16, kcofs[u], so, 0, 0);
    } else if (vlane) {
      const uint32_t so = (uint32_t)s * vss + j0 * vrs;
#pragma unroll
      for (int u = 0; u < 4; ++u)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_u32s*)(dst + kSbKTile + 1024 * u), 16, vcofs[u], so, 0, 0);
    }
  };

  // ---- bias: lane (li, hf) loads keys 16c + 8hf .. +7 of query q0 + li, c = 0, 1 ----
  const uint32_t brs = (uint32_t)a.bias_s[3] * 2;
  const uint32_t bofs = (uint32_t)(q0 + li) * brs + (uint32_t)(kbeg + 8 * hf) * 2;
  // As inline assembly: the compiler cannot track these loads across the unrolled tiles and put
  // a wait for the loads just issued in front of a seed MFMA; the tile-end waits cover them.
  const uint64_t bb64 = reinterpret_cast<uint64_t>(bbase);
  const u32x4 rbw = {(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)bb64),
                     (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(bb64 >> 32) & 0xffff),
                     (uint32_t)__builtin_amdgcn_readfirstlane((int)args.bias_bytes), kRsrcWord3};
  auto load_bias = [&](int t, u32x4 (&bb)[2]) __attribute__((always_inline)) {
    const uint32_t so = (uint32_t)(t * kSbKT) * 2;
    asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(bb[0]) : "v"(bofs), "s"(rbw), "s"(so) : "memory");
    asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen offset:32" : "=v"(bb[1]) : "v"(bofs), "s"(rbw), "s"(so) : "memory");
  };
  // identity operands: row li, k = 8 hf + e of chunk c -> 1 where li == 16c + 8hf + e
  bf16x8 idn[2];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) idn[c][e] = (__bf16)(li == 16 * c + 8 * hf + e ? 1.0f : 0.0f);

  // ---- key-mask bits [K / 32] words, bit i of word w = key 32 w + i valid ----
  uint32_t* mwords = reinterpret_cast<uint32_t*>(smem + kSbMaskOff);
  const bool has_mask = a.mask_k != nullptr;
  if (has_mask) {
    for (int j0 = 64 * wave; j0 < K; j0 += 256) {
      const int j = j0 + lane;
      const uint64_t bits = __ballot(a.mask_k[(int64_t)j * a.mk_s[2]] != 0);
      if (lane < 2) mwords[(j0 >> 5) + lane] = (uint32_t)(bits >> (32 * lane));
    }
  }
  // ---- constant rows of every V tile: piece 6 = (1, 0, ..., 0), piece 7 = 0 ----
  for (int r = tid; r < 2 * 2 * kSbR * kSbKT; r += 256) {
    const int key = r & 31, tileid = r >> 5;             // tileid = (stage, kh, s)
    uint8_t* row = smem + (tileid / (2 * kSbR)) * kSbStage + (tileid % (2 * kSbR)) * kSbPair + kSbKTile + key * kSbVRow;
    const int f = (key & 2) << 1;
    *reinterpret_cast<u32x4*>(row + 16 * (6 ^ f)) = u32x4{0x3f80u, 0u, 0u, 0u};
    *reinterpret_cast<u32x4*>(row + 16 * (7 ^ f)) = u32x4{0u, 0u, 0u, 0u};
  }

  // ---- Q' operands: lane (li, hf), k-step kk: dims 16kk + 8hf .. +7 of query q0 + li, times
  //      scale * log2 e, rounded to bf16 ----
  const float cs = a.scale * SF_LOG2E;
  bf16x8 qop[kSbR][3];
#pragma unroll
  for (int s = 0; s < kSbR; ++s) {
    const uint16_t* qp = (const uint16_t*)a.q + (int64_t)s * a.q_s[0] + (int64_t)(q0 + li) * a.q_s[2] +
                         (int64_t)h * a.q_s[3] + 8 * hf;
#pragma unroll
    for (int kk = 0; kk < 3; ++kk) {
      const u32x4 w = ld16(qp + 16 * kk);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bf16x2 p = cvt_bf2(bflo(w[e]) * cs, bfhi(w[e]) * cs);
        qop[s][kk][2 * e] = p[0];
        qop[s][kk][2 * e + 1] = p[1];
      }
    }
  }

  // ---- per-lane LDS read offsets ----
  // K operand: key li, piece 2kk + hf at position (2kk + hf) ^ ((li >> 3) & 1)
  const uint32_t kread = (uint32_t)li * kSbKRow + 16u * (uint32_t)(hf ^ ((li >> 3) & 1));
  // V^T operand (ds_read_b64_tr_b16): source lane (grp, gi) reads key 16c + 8rd + 4(grp >> 1) +
  // (gi >> 2), dims 32db + 16(grp & 1) + 4(gi & 3) .. +3; piece 4db + 2(grp & 1) + (gi & 3) / 2
  // sits at position piece ^ f, f = (key & 2) << 1 = ((gi >> 3) & 1) * 4
  const int vkey = 4 * (grp >> 1) + (gi >> 2);
  const int vp = 2 * (grp & 1) + ((gi & 3) >> 1);
  const int vfb = (gi >> 3) & 1;
  const uint32_t vcommon = (uint32_t)vkey * kSbVRow + 16u * vp + 8u * (gi & 1);
  const uint32_t vread0 = vcommon + 64u * vfb;            // db = 0: position vp + 4 fb
  const uint32_t vread1 = vcommon + 64u * (1 - vfb);      // db = 1: position vp + 4 (1 - fb)

  const uint32_t lds_base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)smem;
  f32x16 o[kSbR][2];
#pragma unroll
  for (int s = 0; s < kSbR; ++s)
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[s][d][r] = 0.f;

  // ---- pipeline: tile t in stage t & 1; bias loaded three tiles ahead into a 4-slot ring ----
  u32x4 bring[4][2];
#pragma unroll
  for (int s = 0; s < kSbR; ++s) copy_sample(0, 0, s);
#pragma unroll
  for (int p = 0; p < 3; ++p)
    if (p < nt) load_bias(p, bring[p]);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // carried from tile to tile: the P^T and V^T operands of the sample whose P.V is pending
  bf16x8 ppb[2];
  u32x2 part[2][2][2];                                     // [chunk][dim block][read]
  auto tile = [&](int t, auto stage_c, auto slot_c) __attribute__((always_inline)) {
    constexpr int ST = decltype(stage_c)::value, SL = decltype(slot_c)::value;

    // seed: bias^T * log2 e in S^T order; masked keys -inf
    f32x16 seed;
#pragma unroll
    for (int r = 0; r < 16; ++r) seed[r] = 0.f;
    seed = mfma32(idn[0], as_bf16x8(bring[SL][0]), seed);
    seed = mfma32(idn[1], as_bf16x8(bring[SL][1]), seed);
#pragma unroll
    for (int r = 0; r < 16; ++r) seed[r] *= SF_LOG2E;
    if (has_mask) {
      const uint32_t mw = __builtin_amdgcn_readfirstlane(mwords[(kbeg >> 5) + t]);
      if (mw != 0xffffffffu) {
        asm volatile("" ::: "memory");                  // a real branch: not computed on every tile
        const uint32_t mine = mw >> (4 * hf);
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (!((mine >> (8 * (r >> 2) + (r & 3))) & 1u)) seed[r] = -INFINITY;
      }
    }
    // Samples are software-pipelined.  Step s: wait for the K operands of sample s + 1 and the
    // V^T operands of sample s (issued a step earlier), issue the S^T MFMAs of sample s + 1 and
    // the K reads of sample s + 2, then the exponentials and P.V MFMAs of sample s, then the V^T
    // reads of sample s + 1.  All LDS reads of the loop are inline assembly with explicit waits
    // (the compiler issued the K reads one at a time, each behind its own wait).
    const uint32_t stage_lds = lds_base + (uint32_t)(ST * kSbStage + kh * kSbR * kSbPair);
    auto kreads = [&](int s, u32x4 (&kop)[3]) __attribute__((always_inline)) {
      const uint32_t ka = stage_lds + (uint32_t)(s * kSbPair) + kread;
      kop[0] = ds_read16_off<0>(ka);
      kop[1] = ds_read16_off<32>(ka);
      kop[2] = ds_read16_off<64>(ka);
    };
    auto vreads = [&](int s, u32x2 (&part)[2][2][2]) __attribute__((always_inline)) {
      const uint32_t vt_lds = stage_lds + (uint32_t)(s * kSbPair + kSbKTile);
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        const uint32_t va = vt_lds + (db == 0 ? vread0 : vread1);
        part[0][db][0] = tr_read_off<0>(va);
        part[0][db][1] = tr_read_off<8 * kSbVRow>(va);
        part[1][db][0] = tr_read_off<16 * kSbVRow>(va);
        part[1][db][1] = tr_read_off<24 * kSbVRow>(va);
      }
    };
    f32x16 sc, sn;
    u32x4 kop[2][3];                                       // K operands, by sample parity
    // One wave per SIMD issues in order, so a dependent MFMA stalls everything behind it.  The
    // P.V MFMAs therefore run one sample behind: step s interleaves the S^T chain of sample s + 1,
    // the exponentials of sample s and the P.V MFMAs of sample s - 1 (whose V^T operands were read
    // at the end of step s - 1).  Sample 4's P.V runs at the start of the next tile, under its
    // first S^T chain.
    auto exps = [&](int c, bf16x8& pbc) __attribute__((always_inline)) {
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const bf16x2 w = cvt_bf2(fast_exp2(sc[8 * c + 2 * e2]), fast_exp2(sc[8 * c + 2 * e2 + 1]));
        pbc[2 * e2] = w[0];
        pbc[2 * e2 + 1] = w[1];
      }
    };
    auto pv = [&](int s, int c, int db) __attribute__((always_inline)) {
      pv1<0>(o[s][db], u32x4{part[c][db][0][0], part[c][db][0][1], part[c][db][1][0], part[c][db][1][1]}, ppb[c]);
    };
    auto wait_part = [&]() __attribute__((always_inline)) {
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(part[0][0][0]), "+v"(part[0][0][1]), "+v"(part[0][1][0]), "+v"(part[0][1][1]),
                     "+v"(part[1][0][0]), "+v"(part[1][0][1]), "+v"(part[1][1][0]), "+v"(part[1][1][1]));
    };
    kreads(0, kop[0]);
    kreads(1, kop[1]);
    asm volatile("s_waitcnt lgkmcnt(3)" : "+v"(kop[0][0]), "+v"(kop[0][1]), "+v"(kop[0][2]));
    __builtin_amdgcn_sched_barrier(0);
    sc = mfma32(as_bf16x8(kop[0][0]), qop[0][0], seed);
    if (t > 0) pv(kSbR - 1, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    sc = mfma32(as_bf16x8(kop[0][1]), qop[0][1], sc);
    if (t > 0) pv(kSbR - 1, 0, 1);
    __builtin_amdgcn_sched_barrier(0);
    sc = mfma32(as_bf16x8(kop[0][2]), qop[0][2], sc);
    if (t > 0) {
      pv(kSbR - 1, 1, 0);
      pv(kSbR - 1, 1, 1);
    }
#pragma unroll
    for (int s = 0; s < kSbR; ++s) {
      const bool nx = s + 1 < kSbR;
      const u32x4 (&kn)[3] = kop[(s + 1) & 1];
      __builtin_amdgcn_sched_barrier(0);
      // the K operands of sample s + 1; from step 1 on, the 8 V^T reads of sample s - 1 issued
      // after them may stay in flight until its P.V MFMAs
      if (nx) {
        if (s == 0) asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(kop[1][0]), "+v"(kop[1][1]), "+v"(kop[1][2]));
        else asm volatile("s_waitcnt lgkmcnt(8)" : "+v"(kop[(s + 1) & 1][0]), "+v"(kop[(s + 1) & 1][1]), "+v"(kop[(s + 1) & 1][2]));
      }
      __builtin_amdgcn_sched_barrier(0);
      if (nx) sn = mfma32(as_bf16x8(kn[0]), qop[s + 1][0], seed);
      __builtin_amdgcn_sched_barrier(0);
      bf16x8 npb[2];
      exps(0, npb[0]);
      __builtin_amdgcn_sched_barrier(0);
      if (s > 0) {
        wait_part();
        pv(s - 1, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (nx) sn = mfma32(as_bf16x8(kn[1]), qop[s + 1][1], sn);
      if (s > 0) pv(s - 1, 0, 1);
      __builtin_amdgcn_sched_barrier(0);
      exps(1, npb[1]);
      __builtin_amdgcn_sched_barrier(0);
      if (s > 0) pv(s - 1, 1, 0);
      __builtin_amdgcn_sched_barrier(0);
      if (nx) sn = mfma32(as_bf16x8(kn[2]), qop[s + 1][2], sn);
      if (s + 2 < kSbR) kreads(s + 2, kop[s & 1]);
      __builtin_amdgcn_sched_barrier(0);
      if (s > 0) pv(s - 1, 1, 1);
      __builtin_amdgcn_sched_barrier(0);
      vreads(s, part);
      // the next tile's copies in the first three steps (samples 0-1, 2-3, 4), so that they land
      // before the tile ends
      if (t + 1 < nt && s < 3) {
        copy_sample(t + 1, ST ^ 1, 2 * s);
        if (2 * s + 1 < kSbR) copy_sample(t + 1, ST ^ 1, 2 * s + 1);
      }
      ppb[0] = npb[0];
      ppb[1] = npb[1];
      sc = sn;
    }
    // the bias three tiles on, last: the tile-end wait below leaves only these in flight
    if (t + 3 < nt) load_bias(t + 3, bring[(SL + 3) & 3]);
    // next tile's copies (and the bias three tiles on) landed; every wave done with this stage
    // (a __syncthreads would wait for the bias loads in flight as well)
    // (waits the compiler sees, so that it adds none of its own before the seed MFMAs)
    if (t + 3 < nt) __builtin_amdgcn_s_waitcnt(0x0072);   // vmcnt(2) lgkmcnt(0)
    else __builtin_amdgcn_s_waitcnt(0x0070);              // vmcnt(0) lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;
  for (int t = 0; t < nt; t += 4) {
    tile(t, S0{}, S0{});
    tile(t + 1, S1{}, S1{});
    tile(t + 2, S0{}, S2{});
    tile(t + 3, S1{}, S3{});
  }

  // the last tile's sample 4 (its V^T operands landed before the tile-end barrier)
  {
    const u32x4 v00 = {part[0][0][0][0], part[0][0][0][1], part[0][0][1][0], part[0][0][1][1]};
    const u32x4 v01 = {part[0][1][0][0], part[0][1][0][1], part[0][1][1][0], part[0][1][1][1]};
    const u32x4 v10 = {part[1][0][0][0], part[1][0][0][1], part[1][0][1][0], part[1][0][1][1]};
    const u32x4 v11 = {part[1][1][0][0], part[1][1][0][1], part[1][1][1][0], part[1][1][1][1]};
    pv1<0>(o[kSbR - 1][0], v00, ppb[0]);
    pv1<0>(o[kSbR - 1][1], v01, ppb[0]);
    pv1<0>(o[kSbR - 1][0], v10, ppb[1]);
    pv1<0>(o[kSbR - 1][1], v11, ppb[1]);
  }
  asm volatile("s_nop 15\n\ts_nop 15" ::: "memory");   // the last accumulator writes (16 passes) land
  // ---- combine the key halves: each wave writes the partial O^T of the samples it does not
  //      own, then finishes its own (kh 0: samples 0, 2, 4; kh 1: 1, 3) ----
  float* partial = reinterpret_cast<float*>(smem);
  auto preg = [&](int s, int r) __attribute__((always_inline)) -> float* {
    return partial + (((qs * kSbR + s) * kSbPartRegs + r) * 64 + lane);
  };
#pragma unroll
  for (int s = 0; s < kSbR; ++s) {
    if ((s & 1) == kh) continue;                          // owned
#pragma unroll
    for (int r = 0; r < 16; ++r) *preg(s, r) = o[s][0][r];
#pragma unroll
    for (int r = 0; r < 9; ++r) *preg(s, 16 + r) = o[s][1][r];
  }
  // gate prefetch for the owned samples: lane (li, hf) dims 8j + 4hf (j < 4) and 32 + 8j + 4hf
  // (sample indices stay compile-time: a runtime index would put the accumulators in memory)
  const bool has_gate = a.gate != nullptr;
  u32x2 gw[kSbR][6];
#pragma unroll
  for (int s = 0; s < kSbR; ++s) {
#pragma unroll
    for (int j = 0; j < 6; ++j) gw[s][j] = u32x2{0x3f803f80u, 0x3f803f80u};
    if ((s & 1) == kh && has_gate) {
      const uint16_t* gp = (const uint16_t*)a.gate + (int64_t)s * a.g_s[0] + (int64_t)(q0 + li) * a.g_s[2] +
                           (int64_t)h * a.g_s[3] + 4 * hf;
#pragma unroll
      for (int j = 0; j < 6; ++j) gw[s][j] = *reinterpret_cast<const u32x2*>(gp + (j < 4 ? 8 * j : 32 + 8 * (j - 4)));
    }
  }
  __syncthreads();
  uint32_t flagged[kSbR];
#pragma unroll
  for (int s = 0; s < kSbR; ++s) {
    flagged[s] = 0;
    if ((s & 1) != kh) continue;                          // uniform
    f32x16 o0 = o[s][0], o1 = o[s][1];
#pragma unroll
    for (int r = 0; r < 16; ++r) o0[r] += *preg(s, r);
#pragma unroll
    for (int r = 0; r < 9; ++r) o1[r] += *preg(s, 16 + r);
    // l: O^T row 48 = register 8 of dim block 1 on lanes hf = 0
    const float l = __shfl(o1[8], li);
    const bool bad = !(l >= 7.888609052210118e-31f && l <= 1.2676506002282294e30f);   // 2^-100, 2^100
    flagged[s] = (uint32_t)__ballot(bad);
    const float inv = 1.0f / l;
    uint16_t* op = (uint16_t*)a.out + (int64_t)s * a.o_s[0] + (int64_t)(q0 + li) * a.o_s[2] +
                   (int64_t)h * a.o_s[3] + 4 * hf;
    if (!bad) {
#pragma unroll
      for (int j = 0; j < 6; ++j) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (j < 4 ? o0[4 * j + e] : o1[4 * (j - 4) + e]) * inv;
        if (has_gate) {
          v[0] *= sigmoidf_(bflo(gw[s][j][0])); v[1] *= sigmoidf_(bfhi(gw[s][j][0]));
          v[2] *= sigmoidf_(bflo(gw[s][j][1])); v[3] *= sigmoidf_(bfhi(gw[s][j][1]));
        }
        *reinterpret_cast<u32x2*>(op + (j < 4 ? 8 * j : 32 + 8 * (j - 4))) =
            u32x2{pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3])};
      }
    }
  }

  // ---- exact recompute of flagged (sample, query) rows: two-pass softmax in fp32 from global
  //      memory, one row per pass of the wave (lane j takes keys j, j + 64, ...) ----
  uint32_t flags_all[kSbR];
#pragma unroll
  for (int s = 0; s < kSbR; ++s) flags_all[s] = __builtin_amdgcn_readfirstlane(flagged[s]);
#pragma unroll 1
  for (int s = kh; s < kSbR; s += 2) {
    uint32_t fl = 0;
#pragma unroll
    for (int s2 = 0; s2 < kSbR; ++s2) fl = s2 == s ? flags_all[s2] : fl;
    while (fl != 0) {
      const int qi = q0 + __builtin_ctz(fl);
      fl &= fl - 1;
      const uint16_t* qp = (const uint16_t*)a.q + (int64_t)s * a.q_s[0] + (int64_t)qi * a.q_s[2] + (int64_t)h * a.q_s[3];
      const uint16_t* kp = (const uint16_t*)a.k + (int64_t)s * a.k_s[0] + (int64_t)h * a.k_s[3];
      const uint16_t* vp = (const uint16_t*)a.v + (int64_t)s * a.v_s[0] + (int64_t)h * a.v_s[3];
      const uint16_t* bp = (const uint16_t*)a.bias + (int64_t)h * a.bias_s[2] + (int64_t)qi * a.bias_s[3];
      float qf[kSbD];
#pragma unroll
      for (int d = 0; d < kSbD; ++d) qf[d] = bf2f(qp[d]);
      auto logit = [&](int j) __attribute__((always_inline)) -> float {
        const uint16_t* kr = kp + (int64_t)j * a.k_s[2];
        float acc = 0.f;
#pragma unroll
        for (int d = 0; d < kSbD; ++d) acc += qf[d] * bf2f(kr[d]);
        return acc * a.scale + bf2f(bp[j]);
      };
      auto valid = [&](int j) __attribute__((always_inline)) -> bool {
        return !has_mask || ((mwords[j >> 5] >> (j & 31)) & 1u);
      };
      float m = -INFINITY;
      for (int j = lane; j < K; j += 64)
        if (valid(j)) m = fmaxf(m, logit(j));
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
      const bool none = m == -INFINITY;                   // every key masked: uniform weights
      float l = 0.f, acc[kSbD];
#pragma unroll
      for (int d = 0; d < kSbD; ++d) acc[d] = 0.f;
      for (int j = lane; j < K; j += 64) {
        const float w = none ? 1.0f : (valid(j) ? __expf(logit(j) - m) : 0.0f);
        l += w;
        const uint16_t* vr = vp + (int64_t)j * a.v_s[2];
#pragma unroll
        for (int d = 0; d < kSbD; ++d) acc[d] += w * bf2f(vr[d]);
      }
      l = wave_sum(l);
      const float inv = 1.0f / l;
      uint16_t* op = (uint16_t*)a.out + (int64_t)s * a.o_s[0] + (int64_t)qi * a.o_s[2] + (int64_t)h * a.o_s[3];
      const uint16_t* gp = has_gate ? (const uint16_t*)a.gate + (int64_t)s * a.g_s[0] + (int64_t)qi * a.g_s[2] +
                                          (int64_t)h * a.g_s[3]
                                    : nullptr;
#pragma unroll
      for (int d = 0; d < kSbD; ++d) {
        const float sum = wave_sum(acc[d]);
        if (lane == d) {
          float x = sum * inv;
          if (gp != nullptr) x *= sigmoidf_(bf2f(gp[d]));
          op[d] = f2bf(x);
        }
      }
    }
  }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
bool al8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7) == 0; }

}  // namespace

// Whether sb_attn_kernel serves these arguments (see the comment at the top), with the reason
// when it does not.
bool sf_sb_attention_ok(const sf_attention_args* a, const char** why) {
  auto no = [&](const char* w) { if (why) *why = w; return false; };
  if (a->B0 != kSbR || a->B1 != 1) return no("the batch is not 5 samples (B0 = 5, B1 = 1)");
  if (a->D != kSbD || a->Dv != kSbD) return no("head dims are not 48");
  if (a->bias == nullptr || a->bias_s[0] != 0) return no("no bias shared by the samples");
  if (a->mask_q != nullptr || a->kv_index != nullptr) return no("query mask or gathered keys");
  if (a->mask_k != nullptr && a->mk_s[0] != 0) return no("the key mask differs between samples");
  if (a->K % 256 != 0 || a->K > kSbMaxK || a->Q % 64 != 0) return no("K not a multiple of 256 up to 4096, or Q not a multiple of 64");
  if (!al16(a->q) || !al16(a->k) || !al16(a->v) || !al16(a->bias) || !al8(a->out) || (a->gate && !al8(a->gate)))
    return no("unaligned q/k/v/bias/out/gate");
  for (int s = 0; s < 4; ++s) {
    if (s != 1 && (a->q_s[s] % 8 || a->k_s[s] % 8 || a->v_s[s] % 8 || a->bias_s[s] % 8)) return no("strides");
    if (s != 1 && (a->o_s[s] % 4 || (a->gate && a->g_s[s] % 4))) return no("output strides");
  }
  if (a->k_s[0] != a->v_s[0] || a->k_s[2] != a->v_s[2]) return no("K and V strides differ");
  const int64_t ext = (int64_t)(a->B0 - 1) * a->k_s[0] * 2 + (int64_t)a->K * a->k_s[2] * 2;
  const int64_t bext = (int64_t)a->Q * a->bias_s[3] * 2;
  if (ext <= 0 || ext >= (1ll << 31) || bext >= (1ll << 31) || a->k_s[0] < 0 || a->k_s[2] <= 0) return no("extents");
  if ((int64_t)a->H * (a->Q / 64) > 0x7fffffff) return no("grid");
  return true;
}

int sf_sb_attention_launch(const sf_attention_args* a, hipStream_t st) {
  SbArgs args{};
  args.a = *a;
  args.qkv_bytes = (uint32_t)((int64_t)(a->B0 - 1) * a->k_s[0] * 2 + (int64_t)a->K * a->k_s[2] * 2);
  args.bias_bytes = (uint32_t)((int64_t)a->Q * a->bias_s[3] * 2);
  const int tasks = a->H * (a->Q / 64);
  args.xcd = tasks % 8 == 0;
  hipLaunchKernelGGL(sb_attn_kernel, dim3(tasks), dim3(256), 0, st, args);
  return sf_check_launch("sb_attn_kernel");
}
