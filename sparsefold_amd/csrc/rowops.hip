// Row-wise kernels around the attention core on gfx950:
//   layer_norm_kernel   LayerNorm / AdaLN rows (primitives.py:471-497, transformer.py:80-96)
//   linear_kernel       bf16 MFMA GEMM with fused bias / sigmoid / row-broadcast multiplier /
//                       residual epilogue and an optional transposed second output
//                       (primitives.py:328-372 Linear.forward; the transposed output emits
//                       pair-bias planes [H, rows] as blocks.py:329 rearranges them)
//   pair_logits_kernel  LN(z) . W -> bias planes in one pass over z (blocks.py:745-749,
//                       transformer.py:430-447 and :655-666); HBM-bound on z and the planes
//   window_gather_kernel key-window gather of atom_layout.convert (atom_layout.py:61-83)
#include <algorithm>
#include <type_traits>

#include "sf_common.h"

namespace {

// ------------------------------------------------------------------------------------
// LayerNorm / AdaLN: one wave per row, 16-byte chunks, fp32 statistics.
// ------------------------------------------------------------------------------------
// LPR lanes per row (C <= 8 * LPR * 4): a wave normalises 64 / LPR rows at once, so narrow
// rows (C = 128: 16 lanes of 16 bytes) keep every lane busy.
template <int LPR>
__global__ __launch_bounds__(256) void layer_norm_kernel(const sf_layer_norm_args a) {
  constexpr int RPW = 64 / LPR;                  // rows per wave
  const int lane = threadIdx.x & 63, sub = lane % LPR;
  const int64_t row = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + lane / LPR;
  const bool live = row < a.M;
  const int C = a.C, nch = C / 8;
  int64_t src = row;                             // x row this row normalises
  bool zero = false;                             // gathered row outside the window: all zeros
  if (a.gather_idx != nullptr && live) {
    const int64_t smp = row / a.gather_rows, r = row - smp * a.gather_rows;
    const int gi = a.gather_idx[r];
    const bool ok = a.gather_mask[r] != 0 && gi >= 0 && gi < a.gather_src_rows;
    src = smp * a.gather_src_rows + (ok ? gi : 0);
    zero = !ok;
  }
  const uint16_t* xp = (const uint16_t*)a.x + (live ? src : 0) * a.x_rs;
  auto group_sum = [](float v) {
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
  };
  // every operand of the row is requested before the statistics need the first one: the
  // affine / modulation loads do not depend on them, so a row costs one memory round trip
  const uint16_t* scp = nullptr;
  const uint16_t* shp = nullptr;
  if (a.scale != nullptr && live) {
    const int64_t crow = row % a.cond_rows;
    scp = (const uint16_t*)a.scale + crow * a.cond_rs;
    shp = (const uint16_t*)a.shift + crow * a.cond_rs;
  }
  u32x4 w[4], sw[4], hw[4];
  float gv[4][8], bv[4][8];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int ch = sub + LPR * t;
    const bool on = live && ch < nch;
    w[t] = (on && !zero) ? ld16(xp + 8 * ch) : u32x4{0, 0, 0, 0};
    if (a.gamma != nullptr) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        gv[t][e] = on ? a.gamma[8 * ch + e] : 0.f;
        bv[t][e] = (on && a.beta) ? a.beta[8 * ch + e] : 0.f;
      }
    }
    if (scp != nullptr) {
      sw[t] = on ? ld16(scp + 8 * ch) : u32x4{0, 0, 0, 0};
      hw[t] = on ? ld16(shp + 8 * ch) : u32x4{0, 0, 0, 0};
    }
  }
  float sum = 0.f;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) sum += bflo(w[t][e]) + bfhi(w[t][e]);
  const float mean = group_sum(sum) / (float)C;
  float sq = 0.f;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    if (sub + LPR * t < nch) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float d0 = bflo(w[t][e]) - mean, d1 = bfhi(w[t][e]) - mean;
        sq += d0 * d0 + d1 * d1;
      }
    }
  }
  const float rstd = rsqrtf(group_sum(sq) / (float)C + a.eps);
  if (!live) return;
  uint16_t* yp = (uint16_t*)a.y + row * a.y_rs;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int ch = sub + LPR * t;
    if (ch >= nch) continue;
    float v[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = (bflo(w[t][e]) - mean) * rstd;
      v[2 * e + 1] = (bfhi(w[t][e]) - mean) * rstd;
    }
    const int c0 = 8 * ch;
    if (a.gamma != nullptr) {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = v[e] * gv[t][e] + bv[t][e];
    }
    if (scp != nullptr) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[2 * e] = v[2 * e] * bflo(sw[t][e]) + bflo(hw[t][e]);
        v[2 * e + 1] = v[2 * e + 1] * bfhi(sw[t][e]) + bfhi(hw[t][e]);
      }
    }
    st16(yp + c0, u32x4{pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]), pack_bf2(v[4], v[5]),
                        pack_bf2(v[6], v[7])});
  }
}

// ------------------------------------------------------------------------------------
// Linear: Y[M,N] = epi(X[M,K] . Wt[N,K]^T).  128x128 block tile, 4 waves of 64x64,
// K in steps of 32 through LDS, v_mfma_f32_32x32x16_bf16.
// ------------------------------------------------------------------------------------
constexpr int kBM = 128, kBN = 128, kBK = 32, kLD = kBK + 8;

__global__ __launch_bounds__(256) void linear_kernel(const sf_linear_args a) {
  __shared__ __attribute__((aligned(16))) uint16_t sA[kBM * kLD];
  __shared__ __attribute__((aligned(16))) uint16_t sB[kBN * kLD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, li = lane & 31;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)blockIdx.x * kBM;
  const int n0 = blockIdx.y * kBN;
  const uint16_t* xp = (const uint16_t*)a.x;
  const uint16_t* wp = (const uint16_t*)a.wt;

  f32x16 acc[2][2];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mb][nb][r] = 0.f;

  for (int k0 = 0; k0 < a.K; k0 += kBK) {
    __syncthreads();
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int t = tid + 256 * it;
      const int r = t >> 2, c8 = (t & 3) * 8;
      const int kk = k0 + c8;
      const int64_t gm = m0 + r;
      const int gn = n0 + r;
      st16(&sA[r * kLD + c8], (gm < a.M && kk < a.K) ? ld16(xp + gm * a.x_rs + kk) : u32x4{0, 0, 0, 0});
      st16(&sB[r * kLD + c8], (gn < a.N && kk < a.K) ? ld16(wp + (int64_t)gn * a.K + kk) : u32x4{0, 0, 0, 0});
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      bf16x8 av[2], bv[2];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
        av[mb] = as_bf16x8(ld16(&sA[(64 * wm + 32 * mb + li) * kLD + 16 * kk + 8 * half]));
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
        bv[nb] = as_bf16x8(ld16(&sB[(64 * wn + 32 * nb + li) * kLD + 16 * kk + 8 * half]));
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = mfma32(av[mb], bv[nb], acc[mb][nb]);
    }
  }

  uint16_t* yp = (uint16_t*)a.y;
  uint16_t* ytp = (uint16_t*)a.yt;
  const uint16_t* rp = (const uint16_t*)a.residual;
  const uint16_t* mp = (const uint16_t*)a.mul;
  const int ycols = a.ycols > 0 ? a.ycols : a.N;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int n = n0 + 64 * wn + 32 * nb + li;
    if (n >= a.N) continue;
    const float bn = a.bias ? a.bias[n] : 0.f;
    const bool tcol = ytp != nullptr && n >= a.tcol0 && n < a.tcol0 + a.tcols;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float v[4];
        const int64_t mbase = m0 + 64 * wm + 32 * mb + 8 * g + 4 * half;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t m = mbase + e;
          float x = acc[mb][nb][4 * g + e] + bn;
          if (m < a.M) {
            if (a.post_sigmoid) x = sigmoidf_(x);
            if (mp) x *= bf2f(mp[(m % a.mul_rows) * a.mul_rs + n]);
            if (rp) x += bf2f(rp[m * a.r_rs + n]);
            if (yp && n < ycols) yp[m * a.y_rs + n] = f2bf(x);
          }
          v[e] = x;
        }
        if (tcol) {
          uint16_t* tp = ytp + (int64_t)(n - a.tcol0) * a.yt_rs;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (mbase + e < a.M) tp[mbase + e] = f2bf(v[e]);
        }
      }
    }
  }
}

// Rows [0, nrows) of a staged fp32 output tile ct (pitch CP floats, BN columns from n0): bias,
// sigmoid, gated pairs, row-broadcast multiplier, residual, bf16 stores of y.  Tile row rl is
// output row m_first + rl; each thread finishes 8 consecutive columns of one row, so residual /
// multiplier rows are read and y rows written as 16-byte pieces.  keep_final writes the final
// values back into ct (for a transposed pass).
template <int BN>
__device__ __forceinline__ void linear_rows(const sf_linear_args& a, float* ct, int CP, int nrows, int64_t m_first,
                                            int n0, int64_t bz, bool keep_final) {
  uint16_t* yp = a.y ? (uint16_t*)a.y + bz * a.y_bs : nullptr;
  const uint16_t* rp = (const uint16_t*)a.residual;
  const uint16_t* mp = (const uint16_t*)a.mul;
  const int ycols = a.ycols > 0 ? a.ycols : a.N;
  const bool rvec = rp && (a.r_rs % 8 == 0) && ((reinterpret_cast<uintptr_t>(rp) & 15) == 0);
  const bool mvec = mp && (a.mul_rs % 8 == 0) && ((reinterpret_cast<uintptr_t>(mp) & 15) == 0);
  const bool yvec = yp && (a.y_rs % 8 == 0) && ((reinterpret_cast<uintptr_t>(yp) & 15) == 0);
  constexpr int CPR = BN / 8;                                 // 8-column pieces per tile row
  static_assert(256 % CPR == 0, "a thread keeps one column piece for all its rows");
  const int tid = threadIdx.x;
  const int cc = tid % CPR;
  const int n = n0 + 8 * cc;                                  // this thread's columns n .. n+7
  const bool full = n + 8 <= a.N;
  float bv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) bv[e] = 0.f;
  if (a.bias && n < a.N) {
    if (full && ((reinterpret_cast<uintptr_t>(a.bias + n) & 15) == 0)) {
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(a.bias + n), b1 = *reinterpret_cast<const f32x4*>(a.bias + n + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) { bv[e] = b0[e]; bv[4 + e] = b1[e]; }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) bv[e] = n + e < a.N ? a.bias[n + e] : 0.f;
    }
  }
  for (int rl = tid / CPR; rl < nrows; rl += 256 / CPR) {
    const int64_t m = m_first + rl;
    if (m >= a.M || n >= a.N) continue;
    float* cv = &ct[rl * CP + 8 * cc];
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = cv[e] + bv[e];
    if (a.glu) {
      // gated pairs: columns 2j (swish) and 2j + 1 of the interleaved weight give output column j;
      // N % 8 == 0 (checked on the host), so the 8 columns are 4 whole pairs
      uint32_t w[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float g0 = v[4 * e] * sigmoidf_(v[4 * e]) * v[4 * e + 1];
        const float g1 = v[4 * e + 2] * sigmoidf_(v[4 * e + 2]) * v[4 * e + 3];
        w[e] = pack_bf2(g0, g1);
      }
      *reinterpret_cast<u32x2*>(yp + m * a.y_rs + n / 2) = u32x2{w[0], w[1]};
      continue;
    }
    if (a.post_sigmoid) {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = sigmoidf_(v[e]);
    }
    if (mp) {
      const uint16_t* mrow = mp + (m % a.mul_rows) * a.mul_rs + n;
      if (mvec && full) {
        const u32x4 w = ld16(mrow);
#pragma unroll
        for (int e = 0; e < 4; ++e) { v[2 * e] *= bflo(w[e]); v[2 * e + 1] *= bfhi(w[e]); }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (n + e < a.N) v[e] *= bf2f(mrow[e]);
      }
    }
    if (rp) {
      const uint16_t* rrow = rp + m * a.r_rs + n;
      if (rvec && full) {
        const u32x4 w = ld16(rrow);
#pragma unroll
        for (int e = 0; e < 4; ++e) { v[2 * e] += bflo(w[e]); v[2 * e + 1] += bfhi(w[e]); }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (n + e < a.N) v[e] += bf2f(rrow[e]);
      }
    }
    if (yp && n < ycols) {
      uint16_t* yrow = yp + m * a.y_rs + n;
      if (yvec && full && n + 8 <= ycols) {
        st16(yrow, u32x4{pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]), pack_bf2(v[4], v[5]), pack_bf2(v[6], v[7])});
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (n + e < a.N && n + e < ycols) yrow[e] = f2bf(v[e]);
      }
    }
    if (keep_final) {
#pragma unroll
      for (int e = 0; e < 8; ++e) cv[e] = v[e];              // final values for the transposed pass
    }
  }
}

// ------------------------------------------------------------------------------------
// Linear, K % 64 == 0: BMxBN tile, 4 waves (2x2), K in steps of 64 double-buffered in LDS
// through direct-to-LDS loads (global_load_lds_dwordx4: lane L fills bytes 16L..16L+15 of a
// 1 KB chunk = 8 rows x 64 k).  Rows are 128 bytes with their 16-byte slots XOR-swizzled by
// (row & 7), so the operand reads of 8 consecutive lanes hit 8 distinct slots.  The product is
// formed transposed (A operand = weight rows), so each lane owns one output row and 4
// consecutive columns per register group: 8-byte epilogue loads and stores.
// ------------------------------------------------------------------------------------
typedef __attribute__((address_space(3))) uint32_t lds_u32_t;

template <int BM, int BN>
__global__ __launch_bounds__(256) void linear64_kernel(const sf_linear_args a) {
  constexpr int ABYTES = BM * 128, BBYTES = BN * 128, BUF = ABYTES + BBYTES;
  constexpr int CHUNKS = BUF / 1024, CPW = CHUNKS / 4;        // 1 KB chunks per wave per step
  constexpr int WR = BM / 2, WC = BN / 2;                     // wave tile
  constexpr int MB = WR / 32, NB = WC / 32;
  constexpr int CP = BN + 4;                                  // fp32 pitch of the staged output tile
  constexpr int SMEM = 2 * BUF > BM * CP * 4 ? 2 * BUF : BM * CP * 4;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, li = lane & 31;
  const int wm = wave >> 1, wn = wave & 1;
  // Batched: workgroup L (x fastest) is assumed to run on XCD L % 8 (round-robin dispatch) and
  // takes tile (L % 8) * total/8 + L / 8, so that every XCD works through a contiguous range of
  // whole batch members and their operands stay in its own L2.  In dispatch order the batched
  // product of 128 planes of 768 x 768 read its operands 5x over from HBM.
  uint64_t bx = blockIdx.x, by = blockIdx.y, bzu = blockIdx.z;
  if (gridDim.z > 1) {
    const uint64_t gx = gridDim.x, gy = gridDim.y, total = gx * gy * gridDim.z;
    if ((total & 7) == 0) {
      const uint64_t L = blockIdx.x + gx * (blockIdx.y + gy * (uint64_t)blockIdx.z);
      const uint64_t t = (L & 7) * (total >> 3) + (L >> 3);
      bx = t % gx; by = (t / gx) % gy; bzu = t / (gx * gy);
    }
  }
  const int64_t m0 = (int64_t)bx * BM;
  const int n0 = (int)by * BN;
  const int64_t bz = (int64_t)bzu;                            // batch member (0 unless batched)
  const uint16_t* xp = (const uint16_t*)a.x + bz * a.x_bs;
  const uint16_t* wp = (const uint16_t*)a.wt + bz * a.w_bs;
  const int rsw = 8 * ((lane & 7) ^ ((lane >> 3) & 7));       // this lane's swizzled source piece
  const int64_t mlast = a.M - 1;
  const int nlast = a.N - 1;

  auto load_step = [&](int k0, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < CPW; ++u) {
      const int c = wave * CPW + u;                            // uniform
      const uint16_t* src;
      if (c < ABYTES / 1024) {
        const int64_t row = min(m0 + c * 8 + (lane >> 3), mlast);
        src = xp + row * a.x_rs + k0 + rsw;
      } else {
        const int row = min(n0 + (c - ABYTES / 1024) * 8 + (lane >> 3), nlast);
        src = wp + (int64_t)row * a.K + k0 + rsw;
      }
      __builtin_amdgcn_global_load_lds(src, (lds_u32_t*)(smem + buf * BUF + c * 1024), 16, 0, 0);
    }
  };
  auto slot = [&](int buf, int region, int row, int piece) __attribute__((always_inline)) -> const uint8_t* {
    return smem + buf * BUF + region + (row * 8 + (piece ^ (row & 7))) * 16;
  };

  f32x16 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mb][nb][r] = 0.f;

  auto compute = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      bf16x8 xa[MB], wb[NB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        xa[mb] = as_bf16x8(ld16(slot(buf, 0, wm * WR + 32 * mb + li, 2 * kk + half)));
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        wb[nb] = as_bf16x8(ld16(slot(buf, ABYTES, wn * WC + 32 * nb + li, 2 * kk + half)));
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = mfma32(wb[nb], xa[mb], acc[mb][nb]);
    }
  };

  const int nsteps = a.K / 64;
  load_step(0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int ks = 0; ks < nsteps; ks += 2) {
    if (ks + 1 < nsteps) load_step((ks + 1) * 64, 1);
    compute(0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (ks + 1 >= nsteps) break;
    if (ks + 2 < nsteps) load_step((ks + 2) * 64, 0);
    compute(1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  // ---- epilogue.  The fp32 tile goes through LDS (the operand buffers are free after the
  //      k-loop's last barrier); then each thread finishes 8 consecutive columns of one row, so
  //      residual / multiplier rows are read and y rows written as 16-byte pieces, 16 threads
  //      per 256-byte row (8-byte stores straight from the MFMA layout hit 32 rows at once).
  //      The same fp32 operations run in the same order per element as before staging. ----
  float* ct = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        *reinterpret_cast<f32x4*>(&ct[(wm * WR + 32 * mb + li) * CP + wn * WC + 32 * nb + 8 * c + 4 * half]) =
            f32x4{acc[mb][nb][4 * c], acc[mb][nb][4 * c + 1], acc[mb][nb][4 * c + 2], acc[mb][nb][4 * c + 3]};
  __syncthreads();
  linear_rows<BN>(a, ct, CP, BM, m0, n0, bz, a.yt != nullptr);
  uint16_t* ytp = (uint16_t*)a.yt;
  if (ytp) {
    // transposed columns [tcol0, tcol0 + tcols): each thread stores 8 consecutive rows of one column
    __syncthreads();
    constexpr int RPC = BM / 8;                               // 8-row pieces per tile column
    for (int t = tid; t < BN * RPC; t += 256) {
      const int nl = t / RPC, rc = t % RPC;
      const int n = n0 + nl;
      if (n >= a.N || n < a.tcol0 || n >= a.tcol0 + a.tcols) continue;
      const int64_t mb0 = m0 + 8 * rc;
      uint16_t* col = ytp + (int64_t)(n - a.tcol0) * a.yt_rs + mb0;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (mb0 + e < a.M) col[e] = f2bf(ct[(8 * rc + e) * CP + nl]);
    }
  }
}

// ------------------------------------------------------------------------------------
// Pair logits: one thread per pair position; the position's C channels stay in
// registers as packed bf16, LN statistics in fp32, then H dot products against
// gamma-folded weights held in LDS ([c][h] so every thread reads the same words).
// ------------------------------------------------------------------------------------
constexpr int kPLMaxC = 128, kPLMaxH = 64;

template <int H, int CM>  // capacities: a.H <= H planes, a.C <= CM channels (C % 8 == 0)
__global__ __launch_bounds__(256) void pair_logits_kernel(const sf_pair_logits_args a) {
  __shared__ float sG[CM * H];        // gamma[c] * w[h][c]   (zero for h >= a.H)
  __shared__ float sS2[H];            // sum_c beta[c] * w[h][c]
  __shared__ int64_t sPl[H];          // element offset of plane h (a.seg / a.group normalised by the host)
  const int C = a.C, Hr = a.H;
  const int64_t P = a.P, seg = a.seg, grp = a.group;
  const uint16_t* wt = (const uint16_t*)a.w_t;
  for (int t = threadIdx.x; t < C * H; t += 256) {
    const int c = t / H, h = t % H;
    sG[t] = h < Hr ? bf2f(wt[h * C + c]) * (a.ln_w ? a.ln_w[c] : 1.f) : 0.f;
  }
  if (threadIdx.x < H) {
    const int h = threadIdx.x;
    float s = 0.f;
    if (a.ln_b && h < Hr)
      for (int c = 0; c < C; ++c) s += a.ln_b[c] * bf2f(wt[h * C + c]);
    sS2[h] = s;
    const int64_t blk = h / grp;
    sPl[h] = blk * grp * P + (h - blk * grp) * seg;
  }
  __syncthreads();
  const uint16_t* z = (const uint16_t*)a.z;
  uint16_t* op = (uint16_t*)a.out;
  const bool narrow = seg <= 0xffffffffll;
  auto load = [&](int64_t p, u32x4 (&x)[CM / 8]) {
    const uint16_t* zp = z + (p < P ? p : 0) * C;
#pragma unroll
    for (int ch = 0; ch < CM / 8; ++ch) x[ch] = (p < P && 8 * ch < C) ? ld16(zp + 8 * ch) : u32x4{0, 0, 0, 0};
  };
  const int64_t stride = (int64_t)gridDim.x * 256;
  int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  u32x4 xn[CM / 8];
  load(p, xn);
  for (; p < P; p += stride) {
    asm volatile("" ::: "memory");            // keep the LDS weight reads inside the loop (no hoisting into VGPRs)
    uint32_t xw[CM / 2];
    float sum = 0.f;
#pragma unroll
    for (int ch = 0; ch < CM / 8; ++ch)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xw[4 * ch + e] = xn[ch][e];
        sum += bflo(xn[ch][e]) + bfhi(xn[ch][e]);          // channels >= C were loaded as zeros
      }
    load(p + stride, xn);
    const float mean = sum / (float)C;
    float sq = 0.f;
#pragma unroll
    for (int e = 0; e < CM / 2; ++e) {
      if (2 * e < C) {
        const float d0 = bflo(xw[e]) - mean, d1 = bfhi(xw[e]) - mean;
        sq += d0 * d0 + d1 * d1;
      }
    }
    const float rstd = rsqrtf(sq / (float)C + 1e-5f);
    float acc[H];
#pragma unroll
    for (int h = 0; h < H; ++h) acc[h] = 0.f;
#pragma unroll
    for (int e = 0; e < CM / 2; ++e) {
      if (2 * e < C) {
        const float x0 = bflo(xw[e]) - mean, x1 = bfhi(xw[e]) - mean;
#pragma unroll
        for (int h = 0; h < H; ++h) acc[h] += x0 * sG[(2 * e) * H + h] + x1 * sG[(2 * e + 1) * H + h];
      }
    }
    int64_t pos;
    if (narrow) {
      const uint32_t u = (uint32_t)((uint64_t)p / (uint32_t)seg);
      pos = (int64_t)u * grp * seg + (p - (int64_t)u * seg);
    } else {
      const int64_t u = p / seg;
      pos = u * grp * seg + (p - u * seg);
    }
#pragma unroll
    for (int h = 0; h < H; ++h)
      if (h < Hr) __builtin_nontemporal_store(f2bf(acc[h] * rstd + sS2[h]), op + sPl[h] + pos);
  }
}

// ------------------------------------------------------------------------------------
// Window gather: one thread per 16-byte chunk of a gathered key row.
// ------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void window_gather_kernel(const sf_window_gather_args a) {
  const int nch = a.C / 8;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)a.S * a.UK * nch;
  if (t >= total) return;
  const int ch = (int)(t % nch);
  const int64_t rowo = t / nch;                 // s * UK + uk
  const int uk = (int)(rowo % a.UK);
  const int s = (int)(rowo / a.UK);
  const int idx = a.idx[uk];
  const bool ok = a.mask[uk] != 0 && idx >= 0 && idx < a.rows;
  u32x4 w = u32x4{0, 0, 0, 0};
  if (ok) w = ld16((const uint16_t*)a.src + ((int64_t)s * a.rows + idx) * a.C + 8 * ch);
  st16((uint16_t*)a.keys + rowo * a.C + 8 * ch, w);
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// ------------------------------------------------------------------------------------
// Pair logits, C = 128.  A workgroup of W waves takes 32 W consecutive positions per
// iteration, one 32-row step per wave: lane (li, half) loads 8 x 16 bytes of position li,
// normalises them straight into MFMA operands, and D = X . Wf^T against the gamma-folded weight
// held in LDS gives lane li = head, registers = 4 consecutive positions.  The D tiles go to an
// LDS tile [64 planes][32 W positions]; after one barrier each wave stores whole 64 W-byte plane
// runs with 16-byte non-temporal stores (the planes are consumed by a later kernel, so they
// bypass L2 and leave it to the z rows).  The next iteration's z rows are loaded before the
// barrier; the tile is double-buffered, so one barrier per tile suffices.  A workgroup reuses
// its normalised operands for G2 tiles of 64 planes (128 planes per z read).
//
// More planes (the Transformer pack has 384) are split over `hgroups` workgroups per position
// worker, each folding its own G2 x 64 weight rows.  The hgroups workgroups of one worker are
// dispatched back to back onto one XCD (workgroup ids b, b+8, b+16, ...), walk the same
// positions in lock-step and so read each z row from HBM once: the repeats hit that XCD's L2.
// The grid holds only as many workgroups as are resident at once, so all of them sweep one
// contiguous window of every plane together.
// ------------------------------------------------------------------------------------
constexpr int kPLWP = 128 + 8;        // LDS pitch (elements) of folded weight rows
constexpr int kPL128MaxH = 1024;
constexpr int kPLWaves = 4;           // waves per workgroup (4 and 8 measure the same)


// HB: 32-plane blocks per tile (NP = 32 HB planes); G2: tiles per workgroup (the normalised z
// operands are reused for G2 * NP planes; H <= G2 * NP * hgroups, and every tile holds a plane
// h < H); SEG: segmented output; VEC: 16-byte stores (P and seg multiples of 8, out 16-byte
// aligned), else 2-byte stores.
//
// No wait covers a store: the z loads are unconditional (positions past P read position 0, their
// operands are zeroed and their planes never stored), the loop is rotated so that the next step's
// rows are normalised after this step's stores, and with VEC the stores are unconditional too
// (a lane whose plane or positions are past the end stores the last valid plane's or chunk's
// bytes again, identical to what its owner stores).  With a branch around a load or a store, or
// the normalisation at the top of the loop, the compiler waited for every store of the previous
// step before normalising the next.
template <int HB, int G2, bool SEG, bool VEC, int W>
__global__ __launch_bounds__(64 * W) void pair_logits128_kernel(const sf_pair_logits_args a, int64_t steps, int hgroups) {
  constexpr int NP = 32 * HB;                 // planes per tile
  constexpr int TPOS = 32 * W;                // positions per tile (one 32-row step per wave)
  constexpr int TP = TPOS + 8;                // LDS pitch of tile rows
  constexpr int LPP = TPOS / 8;               // lanes per plane run (16 bytes each)
  constexpr int PPI = 64 / LPP;               // planes per store instruction
  constexpr int PPW = NP / W;                 // planes stored per wave per tile
  static_assert(PPW % PPI == 0, "tile planes must split evenly over the waves");
  __shared__ __attribute__((aligned(16))) uint16_t sW[G2 * NP * kPLWP];
  __shared__ __attribute__((aligned(16))) uint16_t sT[2][NP * TP];
  __shared__ float sOff[G2 * NP];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, li = lane & 31;
  // grid = hgroups * workers, workers % 8 == 0
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int hg = slot % hgroups;
  const int64_t worker = (int64_t)(slot / hgroups) * 8 + xcd;
  const int64_t workers = gridDim.x / hgroups;
  const int h0 = hg * G2 * NP;
  const int H = a.H;
  const uint16_t* wt = (const uint16_t*)a.w_t;
  // fold: one wave per weight row, lane = 2 channels
  for (int n = wave; n < G2 * NP; n += W) {
    float w0 = 0.f, w1 = 0.f;
    if (h0 + n < H) {
      const uint32_t raw = *reinterpret_cast<const uint32_t*>(wt + (int64_t)(h0 + n) * 128 + 2 * lane);
      w0 = bflo(raw); w1 = bfhi(raw);
    }
    const float g0 = a.ln_w ? a.ln_w[2 * lane] : 1.f, g1 = a.ln_w ? a.ln_w[2 * lane + 1] : 1.f;
    *reinterpret_cast<uint32_t*>(&sW[n * kPLWP + 2 * lane]) = pack_bf2(w0 * g0, w1 * g1);
    const float part = a.ln_b ? a.ln_b[2 * lane] * w0 + a.ln_b[2 * lane + 1] * w1 : 0.f;
    const float tot = wave_sum(part);
    if (lane == 0) sOff[n] = tot;
  }
  __syncthreads();

  const uint16_t* z = (const uint16_t*)a.z;
  uint16_t* out = (uint16_t*)a.out;
  const int64_t P = a.P, seg = a.seg, grp = a.group;
  // element offset of position p inside its plane (plane hp adds blk*grp*P + h*seg)
  auto pos_off = [&](int64_t p) -> int64_t {
    if (!SEG) return p;
    const int64_t u = p / seg;
    return u * grp * seg + (p - u * seg);
  };
  auto load = [&](int64_t step, u32x4 (&x)[8], bool& valid) {
    const int64_t p = step * 32 + li;
    valid = step < steps && p < P;
    const uint16_t* zp = z + (valid ? p : 0) * 128 + 8 * half;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) x[kk] = ld16(zp + 16 * kk);
  };
  // the planes this wave stores: plane row pl = wave * PPW + PPI * i + lane / LPP, chunk lane % LPP
  const int ch = lane % LPP;
  const int64_t wstride = workers * W;
  int64_t base = worker * W;                  // first step of this workgroup's tile
  if (base >= steps) return;                  // uniform over the workgroup
  u32x4 xn[8];
  bool vn;
  load(base + wave, xn, vn);
  bf16x8 xo[8];
  ln128_operands(xn, vn, xo);
  int buf = 0;
  for (; base < steps; base += wstride) {
    const bool more = base + wstride < steps;   // uniform
    bool vnn = false;
    if (more) load(base + wstride + wave, xn, vnn);
#pragma unroll
    for (int g = 0; g < G2; ++g, buf ^= 1) {
    uint16_t* T = sT[buf];
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) {
      f32x16 acc;
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk)
        acc = mfma32(xo[kk], as_bf16x8(ld16(&sW[(g * NP + 32 * hb + li) * kPLWP + 16 * kk + 8 * half])), acc);
      const float off = sOff[g * NP + 32 * hb + li];
      uint16_t* trow = T + (32 * hb + li) * TP + 32 * wave + 4 * half;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        *reinterpret_cast<u32x2*>(trow + 8 * c) =
            u32x2{pack_bf2(acc[4 * c] + off, acc[4 * c + 1] + off), pack_bf2(acc[4 * c + 2] + off, acc[4 * c + 3] + off)};
    }
    lds_only_barrier();
    const int64_t p = base * 32 + 8 * ch;     // first of this lane's 8 positions
    if constexpr (VEC) {
      // the last valid chunk (P is a multiple of 8 and the tile holds a position below P) and the
      // last valid plane of the tile (it holds one)
      const int64_t pc = min(p, P - 8);
      const int chc = (int)((pc - base * 32) >> 3);
      const int plmax = H - 1 - h0 - g * NP;
#pragma unroll
      for (int i = 0; i < PPW / PPI; ++i) {
        const int pl = min(wave * PPW + PPI * i + lane / LPP, plmax);
        const u32x4 v = ld16(T + pl * TP + 8 * chc);
        const int hh = h0 + g * NP + pl;
        const int64_t blk = hh / grp;
        st16_stream(out + blk * grp * P + (hh - blk * grp) * seg + pos_off(pc), v);
      }
    } else {
#pragma unroll
      for (int i = 0; i < PPW / PPI; ++i) {
        const int pl = wave * PPW + PPI * i + lane / LPP;
        const u32x4 v = ld16(T + pl * TP + 8 * ch);
        const int hh = h0 + g * NP + pl;
        if (hh < H && p < P) {
          const int64_t blk = hh / grp;
          uint16_t* op = out + blk * grp * P + (hh - blk * grp) * seg;
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (p + e < P) op[pos_off(p + e)] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
        }
      }
    }
    }
    if (more) ln128_operands(xn, vnn, xo);
  }
}

}  // namespace

extern "C" int sf_hip_layer_norm_fwd(const sf_layer_norm_args* a, void* stream) {
  if (a == nullptr || a->x == nullptr || a->y == nullptr) { sf_set_error("layer_norm: null x/y"); return 1; }
  if (a->M <= 0 || a->C <= 0 || a->C % 8 != 0 || a->C > 2048) {
    sf_set_error("layer_norm: need M > 0 and C a multiple of 8 in [8, 2048] (M=%lld C=%d)", (long long)a->M, a->C);
    return 1;
  }
  if ((a->scale == nullptr) != (a->shift == nullptr) || (a->scale && a->cond_rows <= 0)) {
    sf_set_error("layer_norm: scale and shift must be given together with cond_rows > 0"); return 1;
  }
  if (a->gather_idx && (a->gather_mask == nullptr || a->gather_rows <= 0 || a->gather_src_rows <= 0 ||
                        a->M % a->gather_rows != 0)) {
    sf_set_error("layer_norm: a gather needs gather_mask, gather_rows > 0 dividing M and gather_src_rows > 0");
    return 1;
  }
  if (!al16(a->x) || !al16(a->y) || a->x_rs % 8 || a->y_rs % 8 ||
      (a->scale && (!al16(a->scale) || !al16(a->shift) || a->cond_rs % 8))) {
    sf_set_error("layer_norm: rows must be 16-byte aligned"); return 1;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int nch = a->C / 8;
  auto launch = [&](auto lpr) {
    constexpr int LPR = decltype(lpr)::value;
    const int64_t rows_per_wg = 4 * (64 / LPR);
    hipLaunchKernelGGL(layer_norm_kernel<LPR>, dim3((unsigned)((a->M + rows_per_wg - 1) / rows_per_wg)), dim3(256), 0, st, *a);
  };
  // fewest lanes per row that hold the row in four 16-byte chunks each, widened (up to a wave
  // per row) while the grid would leave most of the 256 CUs idle
  int lpr = nch <= 8 * 4 ? 8 : nch <= 16 * 4 ? 16 : nch <= 32 * 4 ? 32 : 64;
  while (lpr < 64 && (a->M + 4 * (64 / lpr) - 1) / (4 * (64 / lpr)) < 512) lpr *= 2;
  if (lpr == 8) launch(std::integral_constant<int, 8>{});
  else if (lpr == 16) launch(std::integral_constant<int, 16>{});
  else if (lpr == 32) launch(std::integral_constant<int, 32>{});
  else launch(std::integral_constant<int, 64>{});
  return sf_check_launch("layer_norm_kernel");
}

extern "C" int sf_hip_linear_fwd(const sf_linear_args* a, void* stream) {
  if (a == nullptr || a->x == nullptr || a->wt == nullptr || (a->y == nullptr && a->yt == nullptr)) {
    sf_set_error("linear: null x / wt / outputs"); return 1;
  }
  if (a->M <= 0 || a->N <= 0 || a->K <= 0 || a->K % 8 != 0) {
    sf_set_error("linear: need M, N > 0 and K a positive multiple of 8 (M=%lld N=%d K=%d)", (long long)a->M, a->N, a->K);
    return 1;
  }
  if (!al16(a->x) || !al16(a->wt) || a->x_rs % 8) { sf_set_error("linear: x / wt rows must be 16-byte aligned"); return 1; }
  if (a->mul && a->mul_rows <= 0) { sf_set_error("linear: mul_rows must be positive"); return 1; }
  if (a->yt && (a->tcol0 < 0 || a->tcols < 0 || a->tcol0 + a->tcols > a->N)) {
    sf_set_error("linear: transposed column range out of bounds"); return 1;
  }
  const int32_t batch = a->batch > 1 ? a->batch : 1;
  if (batch > 1 && (a->K % 64 != 0 || batch > 65535 || a->yt || a->mul || a->residual || a->y == nullptr ||
                    a->x_bs % 8 || a->w_bs % 8 || a->y_bs < 0)) {
    sf_set_error("linear: the batched form needs K %% 64 == 0, batch <= 65535, 16-byte aligned batch strides and "
                 "no mul / residual / transposed output (K=%d batch=%d)", a->K, a->batch);
    return 1;
  }
  if (a->glu && (a->K % 64 != 0 || a->N % 8 != 0 || a->y == nullptr || a->yt || a->mul || a->residual ||
                 a->post_sigmoid || a->ycols || !al16(a->y) || a->y_rs % 4)) {
    sf_set_error("linear: the gated (glu) form needs K %% 64 == 0, N %% 8 == 0, an 8-byte aligned y with "
                 "y_rs %% 4 == 0, and no mul / residual / sigmoid / transposed output (K=%d N=%d)", a->K, a->N);
    return 1;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (a->K % 64 == 0) {
    // largest tile that still gives >= 512 workgroups (two per CU); else the smallest
    auto tiles = [&](int bm, int bn) { return ((a->M + bm - 1) / bm) * (int64_t)((a->N + bn - 1) / bn) * batch; };
    int bm = 64, bn = 64;
    if (tiles(128, 128) >= 512) bm = 128, bn = 128;
    else if (tiles(64, 128) >= 512) bm = 64, bn = 128;
    const int64_t gm = (a->M + bm - 1) / bm;
    if (gm > 0x7fffffff) { sf_set_error("linear: M too large"); return 1; }
    const dim3 grid((unsigned)gm, (a->N + bn - 1) / bn, (unsigned)batch);
    if (bm == 128) hipLaunchKernelGGL((linear64_kernel<128, 128>), grid, dim3(256), 0, st, *a);
    else if (bn == 128) hipLaunchKernelGGL((linear64_kernel<64, 128>), grid, dim3(256), 0, st, *a);
    else hipLaunchKernelGGL((linear64_kernel<64, 64>), grid, dim3(256), 0, st, *a);
    return sf_check_launch("linear64_kernel");
  }
  const int64_t gm = (a->M + kBM - 1) / kBM;
  if (gm > 0x7fffffff) { sf_set_error("linear: M too large"); return 1; }
  hipLaunchKernelGGL(linear_kernel, dim3((unsigned)gm, (a->N + kBN - 1) / kBN), dim3(256), 0, st, *a);
  return sf_check_launch("linear_kernel");
}

extern "C" int sf_hip_pair_logits_fwd(const sf_pair_logits_args* a, void* stream) {
  if (a == nullptr || a->z == nullptr || a->w_t == nullptr || a->out == nullptr) {
    sf_set_error("pair_logits: null pointers"); return 1;
  }
  const int max_h = a->C == 128 ? kPL128MaxH : kPLMaxH;
  if (a->P <= 0 || a->C <= 0 || a->C % 8 != 0 || a->C > kPLMaxC || a->H <= 0 || a->H > max_h) {
    sf_set_error("pair_logits: need C a multiple of 8 <= %d and 0 < H <= %d (1024 when C = 128) (C=%d H=%d)",
                 kPLMaxC, kPLMaxH, a->C, a->H);
    return 1;
  }
  if (a->seg < 0 || (a->seg > 0 && (a->P % a->seg != 0 || a->group <= 0 || a->H % a->group != 0))) {
    sf_set_error("pair_logits: segmented output needs P %% seg == 0 and H %% group == 0 (P=%lld seg=%lld H=%d group=%d)",
                 (long long)a->P, (long long)a->seg, a->H, a->group);
    return 1;
  }
  if (!al16(a->z)) { sf_set_error("pair_logits: z must be 16-byte aligned"); return 1; }
  sf_pair_logits_args b = *a;
  if (b.seg == 0) { b.seg = b.P; b.group = b.H; }       // plane-major == one segment, one block
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (b.C == 128) {
    const int64_t steps = (b.P + 31) / 32;
    const int hb = b.H <= 32 ? 1 : 2;
    // two 64-plane tiles per workgroup unless the last workgroup's second tile would hold no plane
    // below H (every tile must hold one: the kernel's stores repeat its last valid plane)
    const int g2 = (b.H <= 64 || (b.H - 1) % 128 < 64) ? 1 : 2;
    const int hgroups = (b.H + 32 * hb * g2 - 1) / (32 * hb * g2);
    const bool seg = b.seg != b.P;
    const bool vec = (b.P % 8 == 0) && (b.seg % 8 == 0) && al16(b.out);
    auto launch = [&](auto kernel) {
      // position workers (a multiple of 8): enough for every tile, and no more workgroups than are
      // resident at once
      const int64_t want = ((steps + kPLWaves - 1) / kPLWaves + 7) / 8 * 8;
      const int64_t cap = std::max<int64_t>(
          8, (sf_resident_workgroups(reinterpret_cast<const void*>(kernel), 64 * kPLWaves) / hgroups) / 8 * 8);
      const int64_t workers = std::min(want, cap);
      hipLaunchKernelGGL(kernel, dim3((unsigned)(workers * hgroups)), dim3(64 * kPLWaves), 0, st, b, steps, hgroups);
    };
    auto by_tile = [&](auto vc) {
      constexpr bool V = decltype(vc)::value;
      if (hb == 1 && !seg) launch(pair_logits128_kernel<1, 1, false, V, kPLWaves>);
      else if (hb == 1) launch(pair_logits128_kernel<1, 1, true, V, kPLWaves>);
      else if (g2 == 1 && !seg) launch(pair_logits128_kernel<2, 1, false, V, kPLWaves>);
      else if (g2 == 1) launch(pair_logits128_kernel<2, 1, true, V, kPLWaves>);
      else if (!seg) launch(pair_logits128_kernel<2, 2, false, V, kPLWaves>);
      else launch(pair_logits128_kernel<2, 2, true, V, kPLWaves>);
    };
    if (vec) by_tile(std::true_type{});
    else by_tile(std::false_type{});
    return sf_check_launch("pair_logits128_kernel");
  }
  auto launch = [&](auto kernel) {
    const int64_t want = (b.P + 255) / 256;
    const int64_t cap = sf_resident_workgroups(reinterpret_cast<const void*>(kernel), 256);
    hipLaunchKernelGGL(kernel, dim3((unsigned)std::min(want, cap)), dim3(256), 0, st, b);
  };
  auto by_h = [&](auto cm) {
    constexpr int CM = decltype(cm)::value;
    if (b.H <= 4) launch(pair_logits_kernel<4, CM>);
    else if (b.H <= 8) launch(pair_logits_kernel<8, CM>);
    else if (b.H <= 16) launch(pair_logits_kernel<16, CM>);
    else if (b.H <= 32) launch(pair_logits_kernel<32, CM>);
    else launch(pair_logits_kernel<64, CM>);
  };
  if (b.C <= 16) by_h(std::integral_constant<int, 16>{});
  else if (b.C <= 32) by_h(std::integral_constant<int, 32>{});
  else if (b.C <= 64) by_h(std::integral_constant<int, 64>{});
  else by_h(std::integral_constant<int, 128>{});
  return sf_check_launch("pair_logits_kernel");
}

extern "C" int sf_hip_window_gather_fwd(const sf_window_gather_args* a, void* stream) {
  if (a == nullptr || a->src == nullptr || a->idx == nullptr || a->mask == nullptr || a->keys == nullptr) {
    sf_set_error("window_gather: null pointers"); return 1;
  }
  if (a->S <= 0 || a->rows <= 0 || a->UK <= 0 || a->C <= 0 || a->C % 8 != 0) {
    sf_set_error("window_gather: bad sizes (S=%d rows=%d UK=%d C=%d)", a->S, a->rows, a->UK, a->C); return 1;
  }
  if (!al16(a->src) || !al16(a->keys)) { sf_set_error("window_gather: src/keys must be 16-byte aligned"); return 1; }
  const int64_t total = (int64_t)a->S * a->UK * (a->C / 8);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(window_gather_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, *a);
  return sf_check_launch("window_gather_kernel");
}
