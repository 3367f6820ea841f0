// Triangle attention module (starting / ending node) on gfx950.
//
// Replaces GridSelfAttention.forward (src/sparsefold/model/trunk/blocks.py:293-366 with the
// per-chunk _attention of :270-291).
//
// Fast path (head dim 32, the trunk's C=128 / H=4 configuration), three kernels:
//   1. tri_proj_kernel   one workgroup per (attention row r, 128 positions): LN(z) in LDS
//                        (blocks.py:317), then one MFMA GEMM against [Wq|Wk|Wv|Wg|Wb]
//                        (blocks.py:276-278, :286, :320) whose epilogue writes every operand
//                        in the layout the attention kernel consumes:
//                          Qs  [r][i][h][d]  q * scale * log2(e)   (logits land in log2 units)
//                          Ks  [r][j][h][d]
//                          Vt  [r][h][d][j'] V transposed, keys in PV-MFMA slot order
//                          Gs  [r][i][h][d]  gate logits
//                          Bs  [h][i][j'']   bias * log2(e) in the untransposed orientation
//                                            (blocks.py:329), masked keys = SF_MASKED_LOGIT,
//                                            keys past N = -inf, keys in S^T register order
//                        For the ending node the workgroup walks z's column instead of its row,
//                        so nothing is transposed in memory (blocks.py:345-346, :362-363).
//   2. tri_attn_kernel   one workgroup per (4 rows, head, 32*W queries); K / V^T tiles of 64
//                        keys for the 4 rows double-buffered in LDS; each wave keeps the online
//                        softmax state of its 32 queries for all 4 rows and feeds the bias tile
//                        -- identical for every row -- as the accumulator input of the S^T MFMA,
//                        so bias loads and conversion are paid once per 4 rows; sigmoid gate in
//                        the epilogue, output written at its pair position.
//   3. linear_kernel     out = z + o W_o (blocks.py:291, :366).
// Other head dims use the generic kernels (layer_norm, linear, attention_fwd, linear).
#include <cmath>

#include "sf_common.h"

namespace {
size_t round_up(size_t x) { return (x + 255) & ~(size_t)255; }
int round64(int n) { return (n + 63) & ~63; }

// ---------------------------------------------------------------------------------------
// Key orders inside a 64-key tile.
// S^T register order: lane half h', register a -> key 8*(a/4) + 4*h' + a%4 of a 32-key half.
__host__ __device__ inline int bias_pos64(int j) {
  const int j32 = j & 31;
  return (j & 32) + 16 * ((j32 >> 2) & 1) + 4 * (j32 >> 3) + (j32 & 3);
}
// PV slot order: 16-key chunk c2, lane half h', slot s -> key 16*c2 + 8*(s/4) + 4*h' + s%4.
__host__ __device__ inline int v_pos64(int j) {
  const int k16 = j & 15;
  return (j & 48) + 8 * ((k16 >> 2) & 1) + (k16 & 3) + 4 * (k16 >> 3);
}

struct FastWs {
  uint16_t *q, *k, *vt, *g, *bias, *o;
  size_t bytes;
};

FastWs carve_fast(void* base, int32_t N, int32_t H) {
  const size_t NP = (size_t)round64(N), E = NP * NP * H * 32;
  FastWs w{};
  char* p = (char*)base;
  size_t off = 0;
  w.q = (uint16_t*)(p + off); off += round_up(E * 2);
  w.k = (uint16_t*)(p + off); off += round_up(E * 2);
  w.vt = (uint16_t*)(p + off); off += round_up(E * 2);
  w.g = (uint16_t*)(p + off); off += round_up(E * 2);
  w.bias = (uint16_t*)(p + off); off += round_up(NP * NP * H * 2);
  w.o = (uint16_t*)(p + off); off += round_up((size_t)N * N * H * 32 * 2);
  w.bytes = off;
  return w;
}

// ---------------------------------------------------------------------------------------
// 1. LN + projection
// ---------------------------------------------------------------------------------------
struct TriProjArgs {
  int N, NP, C, H, transpose;
  float qscale;                       // softmax scale * log2(e)
  const uint16_t* z; const uint8_t* seq;
  const float* ln_w; const float* ln_b;
  const uint16_t* w;                  // [4*H*32 + H, C]
  uint16_t *q, *k, *vt, *g, *bias;
};

constexpr int kPB = 128;              // positions per projection workgroup
constexpr int kPC = 128;              // channels (C) handled by the fast path
constexpr int kXP = kPC + 8;          // LDS pitch (elements) of the normalised tile / weight tile

__global__ __launch_bounds__(256) void tri_proj_kernel(const TriProjArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t sX[kPB * kXP];
  __shared__ __attribute__((aligned(16))) uint16_t sW[128 * kXP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, li = lane & 31;
  const int r = blockIdx.y, p0 = blockIdx.x * kPB;
  const int N = a.N, NP = a.NP, H = a.H;
  const int HD = H * 32;

  // ---- LN of 128 positions; two threads per position, 64 channels each ----
  {
    const int pl = tid >> 1, hc = tid & 1;
    const int p = p0 + pl;
    const int za = a.transpose ? p : r, zb = a.transpose ? r : p;
    const bool valid = za < N && zb < N;
    u32x4 w[8];
    float sum = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      w[t] = valid ? ld16(a.z + ((int64_t)za * N + zb) * kPC + 64 * hc + 8 * t) : u32x4{0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 4; ++e) sum += bflo(w[t][e]) + bfhi(w[t][e]);
    }
    sum += __shfl_xor(sum, 1);
    const float mean = sum * (1.0f / kPC);
    float sq = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float d0 = bflo(w[t][e]) - mean, d1 = bfhi(w[t][e]) - mean;
        sq += d0 * d0 + d1 * d1;
      }
    sq += __shfl_xor(sq, 1);
    const float rstd = rsqrtf(sq * (1.0f / kPC) + 1e-5f);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int c0 = 64 * hc + 8 * t;
      float v[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[2 * e] = (bflo(w[t][e]) - mean) * rstd;
        v[2 * e + 1] = (bfhi(w[t][e]) - mean) * rstd;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = v[e] * a.ln_w[c0 + e] + (a.ln_b ? a.ln_b[c0 + e] : 0.f);
      u32x4 o = u32x4{pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]), pack_bf2(v[4], v[5]), pack_bf2(v[6], v[7])};
      if (!valid) o = u32x4{0, 0, 0, 0};
      st16(&sX[pl * kXP + c0], o);
    }
  }

  // ---- GEMM over 5 column tiles: q, k, v, g (128 columns each = 4 heads x 32), bias ----
  for (int nt = 0; nt < 5; ++nt) {
    const int ncols = nt < 4 ? HD : 32;          // bias tile: H valid rows, rest zero
    __syncthreads();
    for (int t = tid; t < ncols * (kPC / 8); t += 256) {
      const int n = t / (kPC / 8), c8 = (t % (kPC / 8)) * 8;
      u32x4 w = u32x4{0, 0, 0, 0};
      if (nt < 4) w = ld16(a.w + (int64_t)(nt * HD + n) * kPC + c8);
      else if (n < H) w = ld16(a.w + (int64_t)(4 * HD + n) * kPC + c8);
      st16(&sW[n * kXP + c8], w);
    }
    __syncthreads();
    const int nblk = ncols / 32;
    f32x16 acc[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[nb][e] = 0.f;
#pragma unroll
    for (int kk = 0; kk < kPC / 16; ++kk) {
      const bf16x8 av = as_bf16x8(ld16(&sX[(32 * wave + li) * kXP + 16 * kk + 8 * half]));
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        if (nb < nblk) acc[nb] = mfma32(av, as_bf16x8(ld16(&sW[(32 * nb + li) * kXP + 16 * kk + 8 * half])), acc[nb]);
    }
    // ---- epilogue: lane owns column n = 32*nb + li; rows m = 32*wave + 8*(e/4) + 4*half + e%4 ----
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      if (nb >= nblk) continue;
      const int n = 32 * nb + li;               // within the tile: head nb, dim li (q/k/v/g)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int pb = p0 + 32 * wave + 8 * c + 4 * half;   // 4 consecutive positions pb..pb+3
        if (pb >= NP) continue;                              // NP % 4 == 0: all four past the end
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[nb][4 * c + e];
        if (nt == 0 || nt == 1 || nt == 3) {
          uint16_t* dst = nt == 0 ? a.q : (nt == 1 ? a.k : a.g);
          const float sc = nt == 0 ? a.qscale : 1.0f;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            dst[((int64_t)r * NP + pb + e) * HD + n] = f2bf(v[e] * sc);
        } else if (nt == 2) {
          // V^T[r][h][d][v_pos(p)]: 4 consecutive positions stay contiguous
          const int64_t base = (((int64_t)r * H + nb) * 32 + li) * NP + (pb & ~63) + v_pos64(pb & 63);
          *reinterpret_cast<u32x2*>(a.vt + base) = u32x2{pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3])};
        } else if (li < H) {
          // bias plane of head li at untransposed (za, zb)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int p = pb + e;
            const int za = a.transpose ? p : r, zb = a.transpose ? r : p;
            float b = v[e] * SF_LOG2E;
            if (zb >= N) b = -INFINITY;
            else if (za >= N) b = 0.f;
            else if (a.seq[zb] == 0) b = SF_MASKED_LOGIT;
            a.bias[((int64_t)li * NP + za) * NP + (zb & ~63) + bias_pos64(zb & 63)] = f2bf(b);
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// 2. attention
// ---------------------------------------------------------------------------------------
struct TriAttnArgs {
  int N, NP, H, transpose;
  const uint16_t *q, *k, *vt, *g, *bias;
  const uint8_t* seq;
  uint16_t* o;                        // [N][N][H][32] at pair positions
};

constexpr int kTR = 4;                // rows per workgroup
constexpr int kKT = 64;               // keys per tile
constexpr int kKP = 40;               // K tile row pitch (elements): 32 + 8
constexpr int kVP = 72;               // V^T tile row pitch (elements): 64 + 8
constexpr int kKTile = kTR * kKT * kKP;   // elements per K tile buffer
constexpr int kVTile = kTR * 32 * kVP;    // elements per V^T tile buffer

template <int W>
__global__ __launch_bounds__(64 * W) void tri_attn_kernel(const TriAttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t sK[2 * kKTile];
  __shared__ __attribute__((aligned(16))) uint16_t sV[2 * kVTile];
  constexpr int NT = 64 * W;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, li = lane & 31;
  const int N = a.N, NP = a.NP, H = a.H, HD = H * 32;

  // ---- workgroup -> (head, row group, query block); XCD-major so that the workgroups an XCD
  //      runs together share the head's bias plane and the row group's K/V tiles in its L2 ----
  const int QB = (NP + 32 * W - 1) / (32 * W), RG = NP / kTR;
  const int total = QB * RG * H;
  int t = blockIdx.x;
  if ((total & 7) == 0) t = (t & 7) * (total >> 3) + (t >> 3);
  const int qb = t % QB;
  const int rg = (t / QB) % RG;
  const int h = t / (QB * RG);
  const int r0 = rg * kTR;
  const int i = qb * 32 * W + 32 * wave + li;      // this lane's query
  const int iq = min(i, NP - 1);                    // operand row for loads (results of i >= N unused)

  // Q operands (B of S^T = K Q^T) for the 4 rows, row masks
  bf16x8 qb8[kTR][2];
  bool rvalid[kTR], rmasked[kTR];
#pragma unroll
  for (int rr = 0; rr < kTR; ++rr) {
    const int r = r0 + rr;
    rvalid[rr] = r < N;
    rmasked[rr] = rvalid[rr] && a.seq[r] == 0;
    const uint16_t* qp = a.q + (((int64_t)r * NP + iq) * H + h) * 32;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) qb8[rr][kk] = as_bf16x8(ld16(qp + 16 * kk + 8 * half));
  }
  f32x16 o[kTR];
  float m[kTR], l[kTR];
#pragma unroll
  for (int rr = 0; rr < kTR; ++rr) {
#pragma unroll
    for (int e = 0; e < 16; ++e) o[rr][e] = 0.f;
    m[rr] = -INFINITY;
    l[rr] = 0.f;
  }

  // tile loader: 4 rows x (K 64x32 + V^T 32x64) bf16 = 2 x 2048 16-byte chunks
  constexpr int CH = 2 * kTR * 256;
  constexpr int PER = CH / NT;
  u32x4 stage[PER];
  auto load_tile = [&](int j0) {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int c = tid + u * NT;
      const int isv = c >= kTR * 256;
      const int cc = c - isv * kTR * 256;
      const int rr = cc >> 8, w = cc & 255;
      const int r = min(r0 + rr, NP - 1);
      if (!isv) {   // K: key w/4, dims 8*(w%4)
        stage[u] = ld16(a.k + (((int64_t)r * NP + j0 + (w >> 2)) * H + h) * 32 + 8 * (w & 3));
      } else {      // V^T: dim w/8, keys 8*(w%8)
        stage[u] = ld16(a.vt + (((int64_t)r * H + h) * 32 + (w >> 3)) * NP + j0 + 8 * (w & 7));
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int c = tid + u * NT;
      const int isv = c >= kTR * 256;
      const int cc = c - isv * kTR * 256;
      const int rr = cc >> 8, w = cc & 255;
      if (!isv) st16(&sK[buf * kKTile + (rr * kKT + (w >> 2)) * kKP + 8 * (w & 3)], stage[u]);
      else st16(&sV[buf * kVTile + (rr * 32 + (w >> 3)) * kVP + 8 * (w & 7)], stage[u]);
    }
  };
  const uint16_t* bp = a.bias + ((int64_t)h * NP + iq) * NP + 16 * half;

  load_tile(0);
  store_tile(0);
  __syncthreads();
  const int ntiles = NP / kKT;
  for (int tt = 0; tt < ntiles; ++tt) {
    const int buf = tt & 1;
    const int j0 = tt * kKT;
    if (tt + 1 < ntiles) load_tile(j0 + kKT);
    // bias tile -> fp32 accumulator seed, shared by the 4 rows
    f32x16 bseed[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const u32x4 b0 = ld16(bp + j0 + 32 * kb), b1 = ld16(bp + j0 + 32 * kb + 8);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        bseed[kb][2 * e] = bflo(b0[e]);
        bseed[kb][2 * e + 1] = bfhi(b0[e]);
        bseed[kb][8 + 2 * e] = bflo(b1[e]);
        bseed[kb][8 + 2 * e + 1] = bfhi(b1[e]);
      }
    }
#pragma unroll
    for (int rr = 0; rr < kTR; ++rr) {
      if (!rvalid[rr]) continue;
      const uint16_t* kt = &sK[buf * kKTile + rr * kKT * kKP];
      f32x16 s[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        s[kb] = bseed[kb];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
          s[kb] = mfma32(as_bf16x8(ld16(&kt[(32 * kb + li) * kKP + 16 * kk + 8 * half])), qb8[rr][kk], s[kb]);
      }
      if (rmasked[rr]) {   // padded token: every key of this row is masked (uniform weights)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 16; ++e) s[kb][e] = (bseed[kb][e] == -INFINITY) ? -INFINITY : SF_MASKED_LOGIT;
      }
      float tmax = s[0][0];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e) tmax = fmaxf(tmax, s[kb][e]);
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
      const float mnew = fmaxf(m[rr], tmax);
      const float alpha = fast_exp2(m[rr] - mnew);
      m[rr] = mnew;
      l[rr] *= alpha;
#pragma unroll
      for (int e = 0; e < 16; ++e) o[rr][e] *= alpha;
      const uint16_t* vt = &sV[buf * kVTile + rr * 32 * kVP];
#pragma unroll
      for (int c2 = 0; c2 < 4; ++c2) {
        const int kb = c2 >> 1, base = 8 * (c2 & 1);
        bf16x8 pb;
#pragma unroll
        for (int sl = 0; sl < 8; ++sl) {
          const float p = fast_exp2(s[kb][base + sl] - mnew);
          l[rr] += p;
          pb[sl] = (__bf16)p;
        }
        o[rr] = mfma32(as_bf16x8(ld16(&vt[li * kVP + 16 * c2 + 8 * half])), pb, o[rr]);
      }
    }
    if (tt + 1 < ntiles) {
      store_tile(buf ^ 1);
    }
    __syncthreads();
  }

  // ---- epilogue: normalise, gate, store at the pair position ----
  if (i >= N) return;
#pragma unroll
  for (int rr = 0; rr < kTR; ++rr) {
    const int r = r0 + rr;
    if (r >= N) continue;
    const float lt = l[rr] + __shfl_xor(l[rr], 32);
    const float inv = 1.0f / lt;
    const uint16_t* gp = a.g + (((int64_t)r * NP + i) * H + h) * 32;
    const int za = a.transpose ? i : r, zb = a.transpose ? r : i;
    uint16_t* op = a.o + (((int64_t)za * N + zb) * H + h) * 32;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int d0 = 8 * c + 4 * half;
      const u32x2 gw = *reinterpret_cast<const u32x2*>(gp + d0);
      const float g0 = bflo(gw[0]), g1 = bfhi(gw[0]), g2 = bflo(gw[1]), g3 = bfhi(gw[1]);
      const float v0 = o[rr][4 * c] * inv * sigmoidf_(g0), v1 = o[rr][4 * c + 1] * inv * sigmoidf_(g1);
      const float v2 = o[rr][4 * c + 2] * inv * sigmoidf_(g2), v3 = o[rr][4 * c + 3] * inv * sigmoidf_(g3);
      *reinterpret_cast<u32x2*>(op + d0) = u32x2{pack_bf2(v0, v1), pack_bf2(v2, v3)};
    }
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

bool fast_path(int32_t C, int32_t H, int32_t D) { return C == kPC && D == 32 && H * D == kPC; }

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
  return fast_path(C, H, D) ? carve_fast(nullptr, N, H).bytes : carve(nullptr, N, C, H, D).bytes;
}

namespace {
int triangle_fast(const sf_triangle_args* a, void* workspace, size_t workspace_bytes, hipStream_t st, int stages) {
  const int32_t N = a->N, H = a->H;
  const FastWs ws = carve_fast(workspace, N, H);
  if (workspace == nullptr || workspace_bytes < ws.bytes) {
    sf_set_error("triangle: workspace too small (%zu < %zu bytes)", workspace_bytes, ws.bytes);
    return 1;
  }
  const int NP = round64(N);
  TriProjArgs pa{};
  pa.N = N; pa.NP = NP; pa.C = kPC; pa.H = H; pa.transpose = a->transpose;
  pa.qscale = (1.0f / sqrtf(32.0f)) * SF_LOG2E;
  pa.z = (const uint16_t*)a->z; pa.seq = a->seq_mask; pa.ln_w = a->ln_w; pa.ln_b = a->ln_b;
  pa.w = (const uint16_t*)a->w_qkvgb;
  pa.q = ws.q; pa.k = ws.k; pa.vt = ws.vt; pa.g = ws.g; pa.bias = ws.bias;
  if (stages & SF_TRI_STAGE_PROJECT) {
    hipLaunchKernelGGL(tri_proj_kernel, dim3((NP + kPB - 1) / kPB, NP), dim3(256), 0, st, pa);
    if (int rc = sf_check_launch("tri_proj_kernel")) return rc;
  }

  TriAttnArgs aa{};
  aa.N = N; aa.NP = NP; aa.H = H; aa.transpose = a->transpose;
  aa.q = ws.q; aa.k = ws.k; aa.vt = ws.vt; aa.g = ws.g; aa.bias = ws.bias; aa.seq = a->seq_mask; aa.o = ws.o;
  if (stages & SF_TRI_STAGE_ATTEND) {
    if (NP % 256 == 0) {
      const int total = (NP / 256) * (NP / kTR) * H;
      hipLaunchKernelGGL(tri_attn_kernel<8>, dim3(total), dim3(512), 0, st, aa);
    } else {
      const int total = ((NP + 127) / 128) * (NP / kTR) * H;
      hipLaunchKernelGGL(tri_attn_kernel<4>, dim3(total), dim3(256), 0, st, aa);
    }
    if (int rc = sf_check_launch("tri_attn_kernel")) return rc;
  }
  if (!(stages & SF_TRI_STAGE_OUTPUT)) return 0;

  sf_linear_args op{};
  const int64_t HD = (int64_t)H * 32;
  op.M = (int64_t)N * N; op.N = a->C; op.K = (int32_t)HD;
  op.x = ws.o; op.x_rs = HD; op.wt = a->w_o;
  if (a->add_residual) { op.residual = a->z; op.r_rs = a->C; }
  op.mul_rows = 1;
  op.y = a->out; op.y_rs = a->C;
  return sf_hip_linear_fwd(&op, st);
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
    return triangle_fast(a, workspace, workspace_bytes, reinterpret_cast<hipStream_t>(stream), stages);
  if (stages != SF_TRI_STAGE_ALL) {
    sf_set_error("triangle: single stages are available on the head-dim-32 path only (C=%d H=%d D=%d)", C, H, D);
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
  if (stages <= 0 || (stages & ~SF_TRI_STAGE_ALL)) {
    sf_set_error("triangle: invalid stage mask %d", stages);
    return 1;
  }
  return triangle_run(a, workspace, workspace_bytes, stream, stages);
}
