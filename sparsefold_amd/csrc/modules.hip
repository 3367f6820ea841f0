// Module-level entry points: one C call runs a whole attention module's kernel chain against a
// caller-provided workspace (no allocation, one host transition instead of one per kernel).
//
//   sf_hip_self_attention_fwd   SelfAttention.forward (transformer.py:306-345) with AdaLN
//                               (:80-96) and AdaLN-zero (:138-154): single attention with pair
//                               bias (SingleActUpdate's attention, blocks.py:750-763) and the
//                               diffusion-transformer token attention
//   sf_hip_cross_attention_fwd  CrossAttention.forward (transformer.py:549-585), optionally with
//                               the key-window gather of CrossAttTransformer (:671-673)
//   sf_hip_diffusion_conditioning_fwd
//                               the AdaLN scale / shift / zero-gate of every conditioned layer of a
//                               diffusion Transformer from its one shared condition
//                               (DiffusionConditioning.cpp:78-222), consumed through the self-attention
//                               entry's pre_scale / pre_shift / pre_zgate
//
// Each stage is one of the library's own op entry points (LayerNorm, linear, attention, window
// gather), so the numerics are exactly those of the op-level path.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <mutex>

#include "sf_common.h"

namespace {

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Bump allocator over the caller's workspace; sizes are checked by the *_workspace_bytes query.
struct Arena {
  char* base;
  size_t off = 0;
  void* take(size_t bytes) {
    void* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  }
};

// LN (gamma / beta) or AdaLN (LN of the condition, sigmoid scale, shift, modulated LN) of x.
// With gidx, the rows of x are gathered as sf_hip_window_gather_fwd would (gmask, grows rows per
// sample of the gathered space, gsrc rows per sample of x).
int adaln(int64_t rows, int C, const void* x, const void* cond, int64_t cond_rows, int Cs,
          const float* ln_w, const float* ln_b, const float* lnc_w, const float* lnc_b,
          const void* w_scale, const float* b_scale, const void* w_shift, Arena& ws, void* y,
          hipStream_t st, const int32_t* gidx = nullptr, const uint8_t* gmask = nullptr, int64_t grows = 0,
          int64_t gsrc = 0) {
  sf_layer_norm_args ln{};
  ln.M = rows; ln.C = C; ln.eps = 1e-5f;
  ln.x = x; ln.x_rs = C; ln.y = y; ln.y_rs = C;
  ln.gather_idx = gidx; ln.gather_mask = gmask; ln.gather_rows = grows; ln.gather_src_rows = gsrc;
  if (cond == nullptr) {
    ln.gamma = ln_w; ln.beta = ln_b;
    return sf_hip_layer_norm_fwd(&ln, st);
  }
  void* cln = ws.take((size_t)cond_rows * Cs * 2);
  void* scale = ws.take((size_t)cond_rows * C * 2);
  void* shift = ws.take((size_t)cond_rows * C * 2);
  sf_layer_norm_args lc{};
  lc.M = cond_rows; lc.C = Cs; lc.eps = 1e-5f;
  lc.x = cond; lc.x_rs = Cs; lc.gamma = lnc_w; lc.beta = lnc_b; lc.y = cln; lc.y_rs = Cs;
  int rc = sf_hip_layer_norm_fwd(&lc, st);
  if (rc) return rc;
  sf_linear_args l{};
  l.M = cond_rows; l.N = C; l.K = Cs; l.x = cln; l.x_rs = Cs; l.mul_rows = 1;
  l.wt = w_scale; l.bias = b_scale; l.post_sigmoid = 1; l.y = scale; l.y_rs = C;
  if ((rc = sf_hip_linear_fwd(&l, st))) return rc;
  l.wt = w_shift; l.bias = nullptr; l.post_sigmoid = 0; l.y = shift;
  if ((rc = sf_hip_linear_fwd(&l, st))) return rc;
  ln.scale = scale; ln.shift = shift; ln.cond_rows = cond_rows; ln.cond_rs = C;
  return sf_hip_layer_norm_fwd(&ln, st);
}

// out = (o W_t2^T) * sigmoid(cond W_zc^T + b_zc) (when cond) + residual (when given)
// A precomputed multiplier pre_mul [cond_rows, C] (row stride pre_rs) replaces the cond GEMM.
int zero_init_out(int64_t rows, int C, int HD, const void* o, const void* cond, int64_t cond_rows, int Cs,
                  const void* w_zc, const float* b_zc, const void* w_t2, const void* residual, void* out,
                  Arena& ws, hipStream_t st, const void* pre_mul = nullptr, int64_t pre_rs = 0) {
  int rc;
  const void* zmul = pre_mul;
  int64_t zrs = pre_mul ? pre_rs : C;
  if (pre_mul == nullptr && cond != nullptr) {
    void* zbuf = ws.take((size_t)cond_rows * C * 2);
    sf_linear_args z{};
    z.M = cond_rows; z.N = C; z.K = Cs; z.x = cond; z.x_rs = Cs; z.mul_rows = 1;
    z.wt = w_zc; z.bias = b_zc; z.post_sigmoid = 1; z.y = zbuf; z.y_rs = C;
    if ((rc = sf_hip_linear_fwd(&z, st))) return rc;
    zmul = zbuf;
  }
  sf_linear_args l{};
  l.M = rows; l.N = C; l.K = HD; l.x = o; l.x_rs = HD; l.wt = w_t2;
  l.mul = zmul; l.mul_rows = zmul ? cond_rows : 1; l.mul_rs = zrs;
  l.residual = residual; l.r_rs = C;
  l.y = out; l.y_rs = C;
  return sf_hip_linear_fwd(&l, st);
}

// ---------------------------------------------------------------------------------------
// The AdaLN conditioning terms of one layer in one launch (transformer.py:80-96, 138-154):
//   scale = sigmoid(LN(c) W_s^T + b_s),  shift = LN(c) W_sh^T,  zgate = sigmoid(c W_zc^T + b_zc)
// with LN(c) the LayerNorm of the condition rows (lnc_w / lnc_b, eps 1e-5), rounded to bf16 as
// the LayerNorm kernel writes it.  It replaces a LayerNorm and three GEMM launches that each
// fill a fraction of the GPU (1024 x 384 -> 768: 4.8 + 6.2 + 6.3 + 6.6 us in the diffusion
// block).  Workgroup (64-row block, 128-channel block, term), 4 waves: the block's condition
// rows -- normalised unless term 2 -- staged in LDS, then wave w forms channels 32 w .. of all 64
// rows as D^T = W c^T (two 32-row accumulators; lane: row li, channels 8 j + 4 half ..), its
// weight rows read once straight from global memory (they stay in L2).  Every load of a
// workgroup -- its weight chunks, condition rows and the LayerNorm affine -- is issued at its
// start: one memory round trip (with the loads after one another, 19 us: a round trip each).
// With 8 waves of 32 x 32 quadrants every weight chunk was read twice per workgroup (21 us).
// ---------------------------------------------------------------------------------------
struct CondTermsArgs {
  int64_t rows; int C, Cs;
  const uint16_t* cond;                       // [rows, Cs]
  const float *lnc_w, *lnc_b;                 // [Cs] (lnc_b may be null)
  const uint16_t *w_scale, *w_shift, *w_zc;   // [C, Cs]
  const float *b_scale, *b_zc;                // [C] or null
  uint16_t *scale, *shift, *zgate;            // [rows, C]
};
constexpr int kCondMaxCs = 384;

__global__ __launch_bounds__(256) void cond_terms_kernel(const CondTermsArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint16_t sA[];   // [64][Cs + 8], then lnc_w, lnc_b (f32)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = lane >> 5, li = lane & 31;
  const int Cs = a.Cs, pitch = Cs + 8, nch = Cs / 8;
  const int term = blockIdx.z;                                  // 0 scale, 1 shift, 2 zgate
  const int64_t r0 = (int64_t)blockIdx.x * 64;
  const int n0 = blockIdx.y * 128;
  float* sG = reinterpret_cast<float*>(sA + 64 * pitch);
  float* sB = sG + Cs;
  // the weight chunks first (they depend on nothing): A operand of D^T = W c^T, lane (half, li)
  // channel nq + li, k = 16 kc + 8 half ..; wave w takes channels 32 w .. for all 64 rows, so
  // every weight chunk is read once per workgroup
  const uint16_t* W = term == 0 ? a.w_scale : term == 1 ? a.w_shift : a.w_zc;
  const int nq = n0 + 32 * wave;
  u32x4 wr[kCondMaxCs / 16];
  {
    const uint16_t* wp = W + (int64_t)(nq + li) * Cs + 8 * half;
#pragma unroll
    for (int kc = 0; kc < kCondMaxCs / 16; ++kc) wr[kc] = 16 * kc < Cs ? ld16(wp + 16 * kc) : u32x4{0, 0, 0, 0};
  }
  // thread (row tid / 4, part tid % 4): chunks of 8 channels part, part + 4, ...
  constexpr int kParts = 4, kChunks = kCondMaxCs / 8 / kParts;
  const int rr = tid >> 2, q = tid & 3;
  u32x4 v[kChunks];
  {
    const uint16_t* cp = a.cond + min(r0 + rr, a.rows - 1) * Cs;
#pragma unroll
    for (int t = 0; t < kChunks; ++t) v[t] = q + kParts * t < nch ? ld16(cp + 8 * (q + kParts * t)) : u32x4{0, 0, 0, 0};
  }
  if (term < 2)                                                 // the LayerNorm's affine, to LDS
    for (int c = 4 * tid; c < Cs; c += 1024) {
      *reinterpret_cast<f32x4*>(sG + c) = *reinterpret_cast<const f32x4*>(a.lnc_w + c);
      *reinterpret_cast<f32x4*>(sB + c) = a.lnc_b ? *reinterpret_cast<const f32x4*>(a.lnc_b + c) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  __syncthreads();
  {
    float mean = 0.f, rstd = 1.f;
    if (term < 2) {
      float sum = 0.f;
#pragma unroll
      for (int t = 0; t < kChunks; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) sum += bflo(v[t][e]) + bfhi(v[t][e]);
      sum += __shfl_xor(sum, 1);
      sum += __shfl_xor(sum, 2);
      mean = sum / (float)Cs;
      float sq = 0.f;
#pragma unroll
      for (int t = 0; t < kChunks; ++t) {
        if (q + kParts * t < nch) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float d0 = bflo(v[t][e]) - mean, d1 = bfhi(v[t][e]) - mean;
            sq += d0 * d0 + d1 * d1;
          }
        }
      }
      sq += __shfl_xor(sq, 1);
      sq += __shfl_xor(sq, 2);
      rstd = rsqrtf(sq / (float)Cs + 1e-5f);
    }
#pragma unroll
    for (int t = 0; t < kChunks; ++t) {
      const int ch = q + kParts * t;
      if (ch >= nch) continue;
      u32x4 y = v[t];
      if (term < 2) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int c = 8 * ch + 2 * e;
          y[e] = pack_bf2((bflo(v[t][e]) - mean) * rstd * sG[c] + sB[c],
                          (bfhi(v[t][e]) - mean) * rstd * sG[c + 1] + sB[c + 1]);
        }
      }
      st16(&sA[rr * pitch + 8 * ch], y);
    }
  }
  __syncthreads();
  const float* bias = term == 0 ? a.b_scale : term == 1 ? nullptr : a.b_zc;
  f32x16 acc[2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
#pragma unroll
  for (int kc = 0; kc < kCondMaxCs / 16; ++kc)
    if (16 * kc < Cs) {
#pragma unroll
      for (int i = 0; i < 2; ++i)                             // rows 32 i + li: two independent chains
        acc[i] = mfma32(as_bf16x8(wr[kc]), as_bf16x8(ld16(sA + (32 * i + li) * pitch + 8 * half + 16 * kc)), acc[i]);
    }
  float bn[4][4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) bn[j][e] = bias ? bias[nq + 8 * j + 4 * half + e] : 0.f;
  uint16_t* outb = term == 0 ? a.scale : term == 1 ? a.shift : a.zgate;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int64_t row = r0 + 32 * i + li;
    if (row >= a.rows) continue;
    uint16_t* out = outb + row * a.C;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = nq + 8 * j + 4 * half;
      float v4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v4[e] = acc[i][4 * j + e] + bn[j][e];
        if (term != 1) v4[e] = sigmoidf_(v4[e]);
      }
      *reinterpret_cast<u32x2*>(out + n) = u32x2{pack_bf2(v4[0], v4[1]), pack_bf2(v4[2], v4[3])};
    }
  }
}

bool cond_terms_ok(int C, int Cs, const void* cond, const void* w_scale, const void* w_shift, const void* w_zc) {
  const uintptr_t al = reinterpret_cast<uintptr_t>(cond) | reinterpret_cast<uintptr_t>(w_scale) |
                       reinterpret_cast<uintptr_t>(w_shift) | reinterpret_cast<uintptr_t>(w_zc);
  return Cs % 16 == 0 && Cs <= kCondMaxCs && C % 128 == 0 && (al & 15) == 0;   // (f32 vectors: torch-aligned)
}

int cond_terms(int64_t rows, int C, int Cs, const void* cond, const float* lnc_w, const float* lnc_b,
               const void* w_scale, const float* b_scale, const void* w_shift, const void* w_zc, const float* b_zc,
               void* scale, void* shift, void* zgate, hipStream_t st) {
  CondTermsArgs t{};
  t.rows = rows; t.C = C; t.Cs = Cs;
  t.cond = static_cast<const uint16_t*>(cond); t.lnc_w = lnc_w; t.lnc_b = lnc_b;
  t.w_scale = static_cast<const uint16_t*>(w_scale); t.w_shift = static_cast<const uint16_t*>(w_shift);
  t.w_zc = static_cast<const uint16_t*>(w_zc); t.b_scale = b_scale; t.b_zc = b_zc;
  t.scale = static_cast<uint16_t*>(scale); t.shift = static_cast<uint16_t*>(shift); t.zgate = static_cast<uint16_t*>(zgate);
  const size_t lds = (size_t)64 * (Cs + 8) * 2 + (size_t)2 * Cs * 4;   // 53 KB at Cs = 384
  hipLaunchKernelGGL(cond_terms_kernel, dim3((unsigned)((rows + 63) / 64), (unsigned)(C / 128), 3), dim3(256), lds, st, t);
  return sf_check_launch("cond_terms_kernel");
}

// attention stage of the self-attention chain: q, k, v, g are column blocks of y [S*N, 4HD]
sf_attention_args self_attn_args(const sf_self_attention_args* a, const void* y, void* o) {
  const int HD = a->H * a->D;
  sf_attention_args t{};
  t.B0 = a->S; t.B1 = 1; t.Q = a->N; t.K = a->N; t.H = a->H; t.D = a->D; t.Dv = a->D;
  t.scale = a->scale > 0.f ? a->scale : 1.0f / std::sqrt((float)a->D);
  const int64_t ys[4] = {(int64_t)a->N * 4 * HD, 0, 4 * HD, a->D};
  const uint16_t* yb = static_cast<const uint16_t*>(y);
  t.q = yb;          for (int i = 0; i < 4; ++i) t.q_s[i] = ys[i];
  t.k = yb + HD;     for (int i = 0; i < 4; ++i) t.k_s[i] = ys[i];
  t.v = yb + 2 * HD; for (int i = 0; i < 4; ++i) t.v_s[i] = ys[i];
  t.gate = yb + 3 * HD; for (int i = 0; i < 4; ++i) t.g_s[i] = ys[i];
  if (a->bias) {
    t.bias = a->bias; t.bias_s[0] = a->bias_s[0]; t.bias_s[1] = 0; t.bias_s[2] = a->bias_s[1]; t.bias_s[3] = a->bias_s[2];
  }
  if (a->mask) { t.mask_k = a->mask; t.mk_s[0] = 0; t.mk_s[1] = 0; t.mk_s[2] = 1; }
  t.out = o; t.o_s[0] = (int64_t)a->N * HD; t.o_s[1] = 0; t.o_s[2] = HD; t.o_s[3] = a->D;
  return t;
}

// attention stage of the cross-attention chain: q, g are column blocks of yq [rows_q, 2HD],
// k, v of yk [rows_k, 2HD]
sf_attention_args cross_attn_args(const sf_cross_attention_args* a, const void* yq, const void* yk, void* o) {
  const int HD = a->H * a->D;
  sf_attention_args t{};
  t.B0 = a->S; t.B1 = a->U; t.Q = a->Qw; t.K = a->Kw; t.H = a->H; t.D = a->D; t.Dv = a->D;
  t.scale = a->scale > 0.f ? a->scale : 1.0f / std::sqrt((float)a->D);
  const uint16_t* qb = static_cast<const uint16_t*>(yq);
  const uint16_t* kb = static_cast<const uint16_t*>(yk);
  const int64_t qs[4] = {(int64_t)a->U * a->Qw * 2 * HD, (int64_t)a->Qw * 2 * HD, 2 * HD, a->D};
  const int64_t ks[4] = {(int64_t)a->U * a->Kw * 2 * HD, (int64_t)a->Kw * 2 * HD, 2 * HD, a->D};
  t.q = qb;      for (int i = 0; i < 4; ++i) t.q_s[i] = qs[i];
  t.gate = qb + HD; for (int i = 0; i < 4; ++i) t.g_s[i] = qs[i];
  t.k = kb;      for (int i = 0; i < 4; ++i) t.k_s[i] = ks[i];
  t.v = kb + HD; for (int i = 0; i < 4; ++i) t.v_s[i] = ks[i];
  if (a->bias) {
    t.bias = a->bias; t.bias_s[0] = 0; t.bias_s[1] = (int64_t)a->H * a->Qw * a->Kw;
    t.bias_s[2] = (int64_t)a->Qw * a->Kw; t.bias_s[3] = a->Kw;
  }
  if (a->mask_q) { t.mask_q = a->mask_q; t.mq_s[0] = 0; t.mq_s[1] = a->Qw; t.mq_s[2] = 1; }
  if (a->mask_k) { t.mask_k = a->mask_k; t.mk_s[0] = 0; t.mk_s[1] = a->Kw; t.mk_s[2] = 1; }
  t.out = o; t.o_s[0] = (int64_t)a->U * a->Qw * HD; t.o_s[1] = (int64_t)a->Qw * HD; t.o_s[2] = HD; t.o_s[3] = a->D;
  return t;
}

// Per-atom plan: q, g from yq [S*A, 2HD]; k, v from ykv [S][A + 1][2HD] (row A of each sample
// is zero), gathered by the window index.
bool cross_prepared(const sf_cross_attention_args* a) { return a->gather_idx != nullptr && a->pre_q_scale != nullptr; }

sf_attention_args cross_prepared_attn_args(const sf_cross_attention_args* a, const void* yq, const void* ykv, void* o) {
  sf_attention_args t = cross_attn_args(a, yq, ykv, o);
  const int HD = a->H * a->D;
  const int64_t A = (int64_t)a->U * a->Qw;
  const int64_t ks[4] = {(A + 1) * 2 * HD, 0, 2 * HD, a->D};
  for (int i = 0; i < 4; ++i) { t.k_s[i] = ks[i]; t.v_s[i] = ks[i]; }
  t.v = static_cast<const uint16_t*>(ykv) + HD;
  t.kv_index = a->gather_idx; t.kv_mask = a->gather_mask; t.kvi_s = a->Kw; t.kv_zero_row = (int32_t)A;
  return t;
}

// zeroes `words` 16-byte pieces of `rows` rows (stride in 16-byte pieces)
__global__ __launch_bounds__(256) void zero_rows_kernel(u32x4* __restrict__ p, int64_t stride, int rows, int words) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= rows * words) return;
  p[(int64_t)(t / words) * stride + t % words] = u32x4{0, 0, 0, 0};
}

// Per-atom AdaLN and the q/g or k/v projection of the key windows (C = 128, 2HD = 256):
//   side 0: hq = LN(x) * q_scale[a] + q_shift[a],  yq[row] = hq W_qg^T + b_qg
//   side 1: hk = LN(x) * k_scale[a] + k_shift[a],  ykv[s][a] = hk W_kv^T,  ykv[s][A] = 0
// (a = row % A, s = row / A).  Persistent: each workgroup serves one side, keeps that side's weight
// (256 rows, pitch 136) and bias in LDS, and walks blocks of 32 rows.  Per block:
//   1. all 512 threads read the block's x, scale and shift rows as contiguous 16-byte pieces
//      (thread t: row t/16, channels 8 (t%16) .. +7; 4 rows per instruction), reduce each row's
//      LayerNorm statistics over its 16 lanes and write the modulated row (bf16, the operand the
//      LayerNorm + linear chain would read) to LDS;
//   2. wave w forms output columns 32w .. 32w+31, D^T = W h^T: lane (li, half) keeps row li,
//      registers 4g .. 4g+3 the columns 8g + 4 half .. +3.
// One side per workgroup halves the weight staging and the LDS (79 KB), so two workgroups share a
// CU; the two sides of a worker run on one XCD (workgroups b and b + 8), so the second reads the
// block's x rows from that XCD's L2.  (Both sides in one workgroup: 20.5 us for 5 x 8192 atoms.)
// No wait covers a store: the next block's rows are requested before step 2 and normalised after
// its stores, the barriers wait for LDS only, and rows past the end load, normalise and store the
// last row again (identical bytes) instead of branching around the stores.
struct Adaln2Args {
  int64_t rows, A; int S, blocks;
  const uint16_t* x;
  const uint16_t *q_scale, *q_shift, *k_scale, *k_shift; int64_t prs;
  const uint16_t *wqg, *wkv; const float* bqg;
  uint16_t *yq, *ykv;
};
constexpr int kA2Pitch = 136;

__global__ __launch_bounds__(512) void adaln2_proj_kernel(const Adaln2Args a) {
  __shared__ __attribute__((aligned(16))) uint16_t sW[256 * kA2Pitch];     // this side's weight
  __shared__ __attribute__((aligned(16))) uint16_t sH[32 * kA2Pitch];      // the block's modulated rows
  __shared__ __attribute__((aligned(16))) float sB[256];                   // b_qg (side 0), else zeros
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, li = lane & 31;
  const int prow = tid >> 4, pc = tid & 15;           // step 1: this thread's row and 8 channels
  // workgroup b: XCD x = b % 8, side (b / 8) % 2, worker 8 (b / 16) + x (grid = 2 x workers,
  // workers a multiple of 8)
  const int side = (blockIdx.x >> 3) & 1;
  const int worker = (int)((blockIdx.x >> 4) << 3) + (int)(blockIdx.x & 7);
  const int workers = (int)gridDim.x >> 1;
  const uint16_t* const wsrc = side ? a.wkv : a.wqg;
  const uint16_t* const scale = side ? a.k_scale : a.q_scale;
  const uint16_t* const shift = side ? a.k_shift : a.q_shift;
  if (tid < 256) sB[tid] = (side == 0 && a.bqg) ? a.bqg[tid] : 0.f;
  {
    u32x4 st[8];                                       // 256 rows x 16 pieces: 8 per thread
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int t = tid + 512 * j, n = t >> 4, c8 = (t & 15) * 8;
      st[j] = ld16(wsrc + n * 128 + c8);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int t = tid + 512 * j, n = t >> 4, c8 = (t & 15) * 8;
      st16(&sW[n * kA2Pitch + c8], st[j]);
    }
  }
  if (side == 1 && worker == 0)                        // the zero row of every sample's K/V block
    for (int e = tid; e < a.S * 32; e += 512)
      st16(a.ykv + ((int64_t)(e >> 5) * (a.A + 1) + a.A) * 256 + 8 * (e & 31), u32x4{0, 0, 0, 0});
  // step 1 loads of a block: x, this side's scale / shift of row prow, channels 8 pc .. +7
  u32x4 lx, ls, lh;
  auto load_rows = [&](int blk) __attribute__((always_inline)) {
    const int64_t row = min((int64_t)blk * 32 + prow, a.rows - 1), at = row % a.A;
    lx = ld16(a.x + row * 128 + 8 * pc);
    ls = ld16(scale + at * a.prs + 8 * pc);
    lh = ld16(shift + at * a.prs + 8 * pc);
  };
  // ---- step 1: LayerNorm statistics over the row's 16 lanes, modulation -> hm ----
  u32x4 hm;
  auto step1 = [&]() __attribute__((always_inline)) {
    float sum = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) sum += bflo(lx[e]) + bfhi(lx[e]);
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) sum += __shfl_xor(sum, m);
    const float mean = sum * (1.0f / 128);
    float sq = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float d0 = bflo(lx[e]) - mean, d1 = bfhi(lx[e]) - mean;
      sq += d0 * d0 + d1 * d1;
    }
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) sq += __shfl_xor(sq, m);
    const float rstd = rsqrtf(sq * (1.0f / 128) + 1e-5f);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float n0 = (bflo(lx[e]) - mean) * rstd, n1 = (bfhi(lx[e]) - mean) * rstd;
      hm[e] = pack_bf2(n0 * bflo(ls[e]) + bflo(lh[e]), n1 * bfhi(ls[e]) + bfhi(lh[e]));
    }
  };
  int blk = worker;
  if (blk >= a.blocks) return;                         // uniform over the workgroup
  load_rows(blk);
  step1();
  for (; blk < a.blocks; blk += workers) {
    lds_only_barrier();                                // the previous block's step 2 is done with sH
    st16(&sH[prow * kA2Pitch + 8 * pc], hm);
    lds_only_barrier();
    const bool more = blk + workers < a.blocks;         // uniform
    if (more) load_rows(blk + workers);                // lands during step 2
    // ---- step 2: this wave's 32 columns ----
    // rows past the end: sH holds the last row's modulated row (load_rows clamps), so their
    // lanes store that row's bytes again
    const int64_t row = (int64_t)blk * 32 + li;
    const int64_t rr = row < a.rows ? row : a.rows - 1;
    const int64_t at = rr % a.A, smp = rr / a.A;
    f32x16 acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      acc = mfma32(as_bf16x8(ld16(&sW[(32 * wave + li) * kA2Pitch + 16 * kk + 8 * half])),
                   as_bf16x8(ld16(&sH[li * kA2Pitch + 16 * kk + 8 * half])), acc);
    // lane half h' holds columns 8g + 4h' .. +3; after one exchange with the partner lane
    // (li, 1 - h') half 0 holds columns 0..15 and half 1 columns 16..31: 32 contiguous bytes
    uint32_t pk[4][2];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c0 = 32 * wave + 8 * g + 4 * half;
      const f32x4 b4 = *reinterpret_cast<const f32x4*>(&sB[c0]);
      pk[g][0] = pack_bf2(acc[4 * g] + b4[0], acc[4 * g + 1] + b4[1]);
      pk[g][1] = pack_bf2(acc[4 * g + 2] + b4[2], acc[4 * g + 3] + b4[3]);
    }
    // (selects by half as bitwise blends of values: a select between array elements became a
    // run-time index into a stack copy of the array)
    const uint32_t hmask = half ? ~0u : 0u;
    auto blend = [&](uint32_t if1, uint32_t if0) __attribute__((always_inline)) { return (if1 & hmask) | (if0 & ~hmask); };
    uint32_t rx[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int w = 0; w < 2; ++w) rx[j][w] = __shfl_xor(blend(pk[j][w], pk[2 + j][w]), 32);
    // half 0: groups 0, 1 = own columns 8g..8g+3, then the partner's 8g+4..8g+7
    // half 1: groups 2, 3 = the partner's 8g..8g+3, then own 8g+4..8g+7
    const u32x4 lo = {blend(rx[0][0], pk[0][0]), blend(rx[0][1], pk[0][1]), blend(pk[2][0], rx[0][0]), blend(pk[2][1], rx[0][1])};
    const u32x4 hi = {blend(rx[1][0], pk[1][0]), blend(rx[1][1], pk[1][1]), blend(pk[3][0], rx[1][0]), blend(pk[3][1], rx[1][1])};
    uint16_t* dst = side ? a.ykv + (smp * (a.A + 1) + at) * 256 : a.yq + rr * 256;
    uint16_t* q = dst + 32 * wave + 16 * half;
    st16(q, lo);
    st16(q + 8, hi);
    if (more) step1();                                 // the next block's rows, after the stores
  }
}

// Stand-in buffer address for sizing queries: the attention route depends on pointer alignment
// only, and every arena slice is 256-byte aligned.
void* const kArenaAligned = reinterpret_cast<void*>(static_cast<uintptr_t>(1) << 20);

// workspace of the self-attention chain (the arena walk below, run without a base)
size_t self_ws(const sf_self_attention_args* a) {
  Arena ws{nullptr};
  const int64_t rows = (int64_t)a->S * a->N;
  const int HD = a->H * a->D;
  const bool cond_gemms = a->cond && !a->pre_scale;   // AdaLN from cond (not precomputed)
  if (cond_gemms) {                          // LN(cond), scale, shift, zgate
    ws.take((size_t)a->N * a->Cs * 2); ws.take((size_t)a->N * a->C * 2); ws.take((size_t)a->N * a->C * 2);
    ws.take((size_t)a->N * a->C * 2);
  }
  ws.take((size_t)rows * a->C * 2);          // h
  ws.take((size_t)rows * 4 * HD * 2);        // q k v g
  ws.take((size_t)rows * HD * 2);            // o
  const sf_attention_args t = self_attn_args(a, kArenaAligned, kArenaAligned);
  ws.take(sf_attention_workspace_bytes(&t));  // key-range slices of the attention
  if (cond_gemms) ws.take((size_t)a->N * a->C * 2);
  return ws.off;
}

size_t cross_ws(const sf_cross_attention_args* a) {
  Arena ws{nullptr};
  const int64_t qrows = (int64_t)a->S * a->U * a->Qw, krows = (int64_t)a->S * a->U * a->Kw;
  const int HD = a->H * a->D;
  if (cross_prepared(a)) {                   // hq, hk, yq, ykv (+ a zero row per sample), o, slices
    const int64_t A = (int64_t)a->U * a->Qw;
    ws.take((size_t)qrows * a->C * 2);
    ws.take((size_t)qrows * a->C * 2);
    ws.take((size_t)qrows * 2 * HD * 2);
    ws.take((size_t)a->S * (A + 1) * 2 * HD * 2);
    ws.take((size_t)qrows * HD * 2);
    const sf_attention_args t = cross_prepared_attn_args(a, kArenaAligned, kArenaAligned, kArenaAligned);
    ws.take(sf_attention_workspace_bytes(&t));
    return ws.off;
  }
  for (int side = 0; side < 2; ++side) {
    const int64_t cr = (int64_t)a->U * (side ? a->Kw : a->Qw);
    ws.take((size_t)cr * a->C * 2); ws.take((size_t)cr * a->C * 2); ws.take((size_t)cr * a->C * 2);
  }
  ws.take((size_t)qrows * a->C * 2);
  ws.take((size_t)krows * a->C * 2);
  ws.take((size_t)qrows * 2 * HD * 2);
  ws.take((size_t)krows * 2 * HD * 2);
  ws.take((size_t)qrows * HD * 2);
  const sf_attention_args t = cross_attn_args(a, kArenaAligned, kArenaAligned, kArenaAligned);
  ws.take(sf_attention_workspace_bytes(&t));
  ws.take((size_t)a->U * a->Qw * a->C * 2);
  return ws.off;
}

}  // namespace

extern "C" size_t sf_hip_self_attention_workspace_bytes(const sf_self_attention_args* a) {
  return a == nullptr ? 0 : self_ws(a);
}

static int self_attention_run(const sf_self_attention_args* a, void* workspace, size_t workspace_bytes,
                              void* stream) {
  if (a == nullptr || a->x == nullptr || a->out == nullptr || a->w_qkvg == nullptr || a->w_t2 == nullptr) {
    sf_set_error("self_attention: x, out, w_qkvg and w_t2 must be non-null"); return 1;
  }
  if (a->S <= 0 || a->N <= 0 || a->C <= 0 || a->H <= 0 || a->D <= 0 || (a->cond && !a->pre_scale && a->Cs <= 0)) {
    sf_set_error("self_attention: sizes must be positive (S=%d N=%d C=%d H=%d D=%d Cs=%d)",
                 a->S, a->N, a->C, a->H, a->D, a->Cs);
    return 1;
  }
  const bool pre = a->pre_scale != nullptr;
  if (pre && (a->pre_shift == nullptr || a->pre_zgate == nullptr || a->pre_rs < a->C)) {
    sf_set_error("self_attention: pre_scale needs pre_shift, pre_zgate and pre_rs >= C (pre_rs=%lld)",
                 (long long)a->pre_rs);
    return 1;
  }
  if (!pre && a->cond && (a->w_scale == nullptr || a->w_shift == nullptr || a->w_zc == nullptr)) {
    sf_set_error("self_attention: a condition needs w_scale, w_shift and w_zc"); return 1;
  }
  if (workspace == nullptr || workspace_bytes < self_ws(a)) {
    sf_set_error("self_attention: workspace of %zu bytes needed, %zu given", self_ws(a), workspace_bytes);
    return 1;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  Arena ws{static_cast<char*>(workspace)};
  const int64_t rows = (int64_t)a->S * a->N;
  const int HD = a->H * a->D;
  void* h = nullptr;
  int rc;
  void *c_scale = nullptr, *c_shift = nullptr, *c_zgate = nullptr;
  const bool fused_cond = a->cond && !pre && cond_terms_ok(a->C, a->Cs, a->cond, a->w_scale, a->w_shift, a->w_zc);
  {
    // the AdaLN workspace is taken first, as in self_ws
    Arena probe = ws;
    if (a->cond && !pre) {
      probe.take((size_t)a->N * a->Cs * 2);
      c_scale = probe.take((size_t)a->N * a->C * 2); c_shift = probe.take((size_t)a->N * a->C * 2);
      c_zgate = probe.take((size_t)a->N * a->C * 2);
    }
    h = probe.take((size_t)rows * a->C * 2);
    if (pre || fused_cond) {
      // the conditioning terms of this layer in one launch (or given), then the modulated LayerNorm
      if (fused_cond && (rc = cond_terms(a->N, a->C, a->Cs, a->cond, a->lnc_w, a->lnc_b, a->w_scale, a->b_scale,
                                         a->w_shift, a->w_zc, a->b_zc, c_scale, c_shift, c_zgate, st))) {
        return rc;
      }
      sf_layer_norm_args ln{};
      ln.M = rows; ln.C = a->C; ln.eps = 1e-5f;
      ln.x = a->x; ln.x_rs = a->C; ln.y = h; ln.y_rs = a->C;
      ln.scale = pre ? a->pre_scale : c_scale; ln.shift = pre ? a->pre_shift : c_shift; ln.cond_rows = a->N;
      ln.cond_rs = pre ? a->pre_rs : a->C;
      if ((rc = sf_hip_layer_norm_fwd(&ln, st))) return rc;
    } else if ((rc = adaln(rows, a->C, a->x, a->cond, a->N, a->Cs, a->ln_w, a->ln_b, a->lnc_w, a->lnc_b,
                           a->w_scale, a->b_scale, a->w_shift, ws, h, st))) {
      return rc;
    }
    ws = probe;
  }
  void* y = ws.take((size_t)rows * 4 * HD * 2);
  void* o = ws.take((size_t)rows * HD * 2);
  sf_linear_args p{};
  p.M = rows; p.N = 4 * HD; p.K = a->C; p.x = h; p.x_rs = a->C; p.wt = a->w_qkvg; p.bias = a->b_qkvg;
  p.mul_rows = 1; p.y = y; p.y_rs = 4 * HD;
  if ((rc = sf_hip_linear_fwd(&p, st))) return rc;
  const sf_attention_args t = self_attn_args(a, y, o);
  const size_t split = sf_attention_workspace_bytes(&t);
  void* split_ws = ws.take(split);
  if ((rc = sf_attention_run(&t, split_ws, split, st))) return rc;
  return zero_init_out(rows, a->C, HD, o, pre || fused_cond ? nullptr : a->cond, a->N, a->Cs, a->w_zc, a->b_zc,
                       a->w_t2, a->add_residual ? a->x : nullptr, a->out, ws, st,
                       pre ? a->pre_zgate : c_zgate, pre ? a->pre_rs : a->C);
}

extern "C" int sf_hip_self_attention_fwd(const sf_self_attention_args* a, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  return self_attention_run(a, workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------------------------------
// Allocation-free variant: the chain's scratch (normalised rows, q/k/v/g, o, key-slice
// partials, AdaLN terms) lives in a fixed device array instead of a caller workspace.  Every
// byte of it that a kernel reads was written earlier in the same call, so nothing needs
// clearing between calls.  Each GPU holds its own copy of the array for the life of the process;
// calls that overlap on one GPU share it and race.
// ---------------------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[SF_HIP_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::once_flag g_scratch_once[kMaxDevices];
hipError_t g_scratch_status[kMaxDevices];
void* g_scratch_addr[kMaxDevices];

// The device address of this GPU's scratch array, looked up once per device with that device
// current (host code must never pass the array's own name to a kernel: it is a host-side stand-in).
int scratch_address(void** addr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    sf_set_error("self_attention_noalloc: no usable current device (%d)", dev);
    return 1;
  }
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    g_scratch_status[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_addr[dev] = g_scratch_status[dev] == hipSuccess ? p : nullptr;
  });
  if (g_scratch_status[dev] != hipSuccess || g_scratch_addr[dev] == nullptr) {
    sf_set_error("self_attention_noalloc: scratch address lookup failed on device %d: %s", dev,
                 hipGetErrorString(g_scratch_status[dev]));
    return 1;
  }
  *addr = g_scratch_addr[dev];
  return 0;
}
}  // namespace

extern "C" int sf_hip_self_attention_fwd_noalloc(const sf_self_attention_args* a, void* stream) {
  if (a == nullptr) { sf_set_error("self_attention_noalloc: null arguments"); return 1; }
  const size_t need = self_ws(a);
  if (need > (size_t)SF_HIP_NOALLOC_SCRATCH_BYTES) {
    sf_set_error("self_attention_noalloc: these sizes need %zu bytes of scratch; the fixed scratch holds %zu "
                 "(use sf_hip_self_attention_fwd with a workspace)", need, (size_t)SF_HIP_NOALLOC_SCRATCH_BYTES);
    return 1;
  }
  void* ws = nullptr;
  if (int rc = scratch_address(&ws)) return rc;
  return self_attention_run(a, ws, SF_HIP_NOALLOC_SCRATCH_BYTES, stream);
}

extern "C" size_t sf_hip_cross_attention_workspace_bytes(const sf_cross_attention_args* a) {
  return a == nullptr ? 0 : cross_ws(a);
}

namespace {
// ---------------------------------------------------------------------------------------
// Window attention and the output stage in one kernel (per-atom plan; 32-query / 128-key
// windows, H = 4, D = 32, C = 128): one workgroup per (sample s, window u), wave h runs head h.
// CrossAttention.forward (transformer.py:549-585) after the q/g, k/v projections:
//   S^T  = K Q^T + bias / scale (+ SF_MASKED_LOGIT for masked keys; a masked query weighs every
//          key equally), K gathered row by row straight into the MFMA A operand
//   P    = 2^(scale log2e (S^T - m)), m the exact maximum over the 128 keys, as bf16; l = sum P
//   O^T  = V^T P^T, the window's 128 V rows of head h copied into LDS (global_load_lds) and read
//          transposed (ds_read_b64_tr_b16)
//   og   = O / l * sigmoid(g) -> LDS [query][h * 32 + d] (over the V rows, after a barrier)
//   out  = og W_t2^T * zgate + x: wave w takes output channels 32w .. 32w + 31
// Against the separate attention and output-projection kernels this drops the o round trip
// (the attention's store and the projection's load) and a launch; every window's bias tile is
// read by its 5 samples from one L2 (task order below).
// ---------------------------------------------------------------------------------------
typedef __attribute__((address_space(3))) uint32_t lds_u32w;
typedef short v4i16w __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16w lds_v4i16w;

struct WinFusedArgs {
  int S, U, A;                          // samples, windows, atoms per sample (= 32 U)
  const uint16_t* yq;                   // [S * A][256]: q (h * 32 + d) | g (128 + h * 32 + d)
  const uint16_t* ykv;                  // [S][A + 1][256]: k | v, row A zero
  const int32_t* gidx; const uint8_t* gmask;   // [U][128] key -> atom, gather mask
  const uint8_t *mask_q, *mask_k;       // [U][32], [U][128] (null: all valid)
  const uint16_t* bias;                 // [U][4][32][128] (null: none)
  const uint16_t* w_t2;                 // [128][128]: output channel x (h * 32 + d)
  const uint16_t* zgate; int64_t zrs;   // [A] rows of 128, row stride zrs
  const uint16_t* x;                    // residual [S * A][128] (null: none)
  uint16_t* out;                        // [S * A][128]
  float scale;                          // logits scale (q.k scale + bias)
};
constexpr int kWinOgPitch = 136;        // og rows in LDS (bf16): 272 bytes apart, conflict-free

// (at most 128 registers: four workgroups per CU)
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void window_attn_out_kernel(const WinFusedArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[4 * 8192];   // V rows per wave, then og
  const int tid = threadIdx.x, lane = tid & 63;
  const int h = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, li = lane & 31;
  // Workgroup b runs on XCD b mod 8: each XCD takes a contiguous run of (window, sample) tasks,
  // so the samples of a window (one bias tile) meet in one L2.
  const int ntask = a.S * a.U, per = ntask >> 3;
  const int task = (int)blockIdx.x < 8 * per ? (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3) : (int)blockIdx.x;
  const int u = task / a.S, s = task - u * a.S;
  const int64_t qrow = (int64_t)s * a.A + 32 * u;            // row of query 0 in yq / x / out
  const uint16_t* kv = a.ykv + (int64_t)s * (a.A + 1) * 256;

  // rows of keys lane and lane + 64: the zero row A for a gather-masked or out-of-range key
  int rowA, rowB;
  {
    const int32_t i0 = a.gidx[(int64_t)u * 128 + lane], i1 = a.gidx[(int64_t)u * 128 + lane + 64];
    const uint8_t m0 = a.gmask[(int64_t)u * 128 + lane], m1 = a.gmask[(int64_t)u * 128 + lane + 64];
    rowA = (m0 == 0 || i0 < 0 || i0 >= a.A) ? a.A : i0;
    rowB = (m1 == 0 || i1 < 0 || i1 >= a.A) ? a.A : i1;
  }
  // V rows of head h -> LDS [key][32 dims] (64 bytes a row): copy c moves keys 16c .. 16c + 15
  uint8_t* vsm = smem + h * 8192;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int key = 16 * c + (lane >> 2);
    const int row = __shfl(c < 4 ? rowA : rowB, key & 63);
    __builtin_amdgcn_global_load_lds(kv + (int64_t)row * 256 + 128 + h * 32 + 8 * (lane & 3),
                                     (lds_u32w*)(vsm + c * 1024), 16, 0, 0);
  }
  // K (A operand of S^T, lane (half, li): key 32 kb + li, dims 16 kk + 8 half ..) and Q (B operand)
  u32x4 kr[4][2];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    const int row = __shfl(kb < 2 ? rowA : rowB, (32 * kb + li) & 63);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) kr[kb][kk] = ld16(kv + (int64_t)row * 256 + h * 32 + 16 * kk + 8 * half);
  }
  const uint16_t* qp = a.yq + (qrow + li) * 256 + h * 32 + 8 * half;
  const bf16x8 qb0 = as_bf16x8(ld16(qp)), qb1 = as_bf16x8(ld16(qp + 16));
  // bias of query li, keys 16 c + 8 half .. + 7: the B operand of an MFMA that adds it to S^T
  // through an identity A (16-byte loads: with the keys of the S^T registers, 8 bytes a lane, the
  // loads were twice as many, each touching as many rows), loaded per key block
  const int64_t boff = (((int64_t)u * 4 + h) * 32 + li) * 128 + 8 * half;   // element offset in bias
  const bool kvalid0 = a.mask_k == nullptr || a.mask_k[(int64_t)u * 128 + lane] != 0;
  const bool kvalid1 = a.mask_k == nullptr || a.mask_k[(int64_t)u * 128 + lane + 64] != 0;
  const uint64_t mk0 = __ballot(kvalid0), mk1 = __ballot(kvalid1);
  const bool qvalid = a.mask_q == nullptr || a.mask_q[(int64_t)u * 32 + li] != 0;

  // ---- S^T = scale K Q^T + bias, masks ----
  // identity chunk c of a 32-key block: A row r, k = 8 half + e is 1 where r = 16 c + 8 half + e
  bf16x8 idn[2];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) idn[c][e] = (__bf16)(li == 16 * c + 8 * half + e ? 1.0f : 0.0f);
  f32x16 sc[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
    for (int r = 0; r < 16; ++r) sc[kb][r] = 0.f;
    sc[kb] = mfma32(as_bf16x8(kr[kb][0]), qb0, sc[kb]);
    sc[kb] = mfma32(as_bf16x8(kr[kb][1]), qb1, sc[kb]);
#pragma unroll
    for (int r = 0; r < 16; ++r) sc[kb][r] *= a.scale;
    if (a.bias != nullptr) {                                // uniform
      sc[kb] = mfma32(idn[0], as_bf16x8(ld16(a.bias + boff + 32 * kb)), sc[kb]);
      sc[kb] = mfma32(idn[1], as_bf16x8(ld16(a.bias + boff + 32 * kb + 16)), sc[kb]);
    }
  }
  if ((mk0 & mk1) != ~0ull) {                               // uniform: some key masked
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      // bit 8 j + i: key 32 kb + 8 j + 4 half + i, S^T register 4 j + i
      const uint32_t mw = (uint32_t)((kb < 2 ? mk0 : mk1) >> (32 * (kb & 1) + 4 * half));
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (((mw >> (8 * (r >> 2) + (r & 3))) & 1u) == 0) sc[kb][r] += SF_MASKED_LOGIT;
    }
  }
  if (!qvalid) {                                            // masked query: every key alike
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[kb][r] = 0.f;
  }
  // ---- P against the exact row maximum ----
  float m = sc[0][0];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int r = 0; r < 16; ++r) m = fmaxf(m, sc[kb][r]);
  m = fmaxf(m, __shfl_xor(m, 32));
  const float mb = m * SF_LOG2E;
  bf16x2 pw[32];
  float l0 = 0.f, l1 = 0.f;
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pw[8 * kb + e] = cvt_bf2(fast_exp2(__builtin_fmaf(sc[kb][2 * e], SF_LOG2E, -mb)),
                               fast_exp2(__builtin_fmaf(sc[kb][2 * e + 1], SF_LOG2E, -mb)));
      if (e & 1) l1 = add_bf2(pw[8 * kb + e], l1); else l0 = add_bf2(pw[8 * kb + e], l0);
    }
  float l = l0 + l1;
  l += __shfl_xor(l, 32);

  // ---- O^T = V^T P^T ----
  __builtin_amdgcn_s_waitcnt(0);                            // this wave's V copies have landed
  asm volatile("" ::: "memory");
  f32x16 o;
#pragma unroll
  for (int r = 0; r < 16; ++r) o[r] = 0.f;
  {
    const int grp = lane >> 4, gi = lane & 15, ekey = gi >> 2, q4 = gi & 3;
    const int d = 16 * (grp & 1) + 4 * q4;
#pragma unroll
    for (int c2 = 0; c2 < 8; ++c2) {
      bf16x8 pb;
#pragma unroll
      for (int q2 = 0; q2 < 4; ++q2) {
        pb[2 * q2] = pw[4 * c2 + q2][0];
        pb[2 * q2 + 1] = pw[4 * c2 + q2][1];
      }
      u32x2 part[2];
#pragma unroll
      for (int rd = 0; rd < 2; ++rd) {
        const int key = 16 * c2 + 8 * rd + 4 * (grp >> 1) + ekey;
        const int off = key * 64 + ((d >> 3) << 4) + ((d >> 2) & 1) * 8;
        part[rd] = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16w*)(vsm + off)));
      }
      o = mfma32(as_bf16x8(u32x4{part[0][0], part[0][1], part[1][0], part[1][1]}), pb, o);
    }
  }
  // 16-byte pieces of 8 dims (channels) per lane -> the 4-dim runs of the O^T registers: lane
  // half 0 loaded dims 0..7 and 16..23, half 1 dims 8..15 and 24..31; run j = dims 8 j + 4 half
  // .. + 3, half of them from the partner lane (l xor 32), exchanged by permlane32_swap
  const uint32_t hm = half ? ~0u : 0u;
  auto blend = [&](uint32_t if1, uint32_t if0) __attribute__((always_inline)) { return (if1 & hm) | (if0 & ~hm); };
  auto runs = [&](const u32x4& p0, const u32x4& p1, u32x2 (&rj)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const u32x4& p = q ? p1 : p0;
      const auto s0 = __builtin_amdgcn_permlane32_swap(p[0], p[2], false, false);
      const auto s1 = __builtin_amdgcn_permlane32_swap(p[1], p[3], false, false);
      // half 0: run 2q = own words 0, 1; run 2q + 1 = the partner's words 0, 1 (s*[1])
      // half 1: run 2q = the partner's words 2, 3 (s*[0]); run 2q + 1 = own words 2, 3
      rj[2 * q] = u32x2{blend(s0[0], p[0]), blend(s1[0], p[1])};
      rj[2 * q + 1] = u32x2{blend(p[2], s0[1]), blend(p[3], s1[1])};
    }
  };
  // gate of query li, dims 8 j + 4 half .. + 3 (O^T registers 4 j .. 4 j + 3), W_t2 rows 32 h +
  // li (A operand of the projection; L2-resident), zero-gate and residual of the output channels
  // 32 h + 8 j + 4 half .. + 3 of query li: issued after P.V, whose P registers they reuse (held
  // through P.V these loads cost more than their latency hidden)
  const uint16_t* gp = a.yq + (qrow + li) * 256 + 128 + h * 32;
  const u32x4 gl0 = ld16(gp + 8 * half), gl1 = ld16(gp + 16 + 8 * half);
  u32x4 wr[8];
  const uint16_t* wp = a.w_t2 + (int64_t)(32 * h + li) * 128 + 8 * half;
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) wr[kk] = ld16(wp + 16 * kk);
  const int64_t orow = qrow + li;
  const uint16_t* zp = a.zgate + (int64_t)(32 * u + li) * a.zrs + 32 * h;
  const u32x4 zl0 = ld16(zp + 8 * half), zl1 = ld16(zp + 16 + 8 * half);
  u32x4 xl0 = u32x4{0, 0, 0, 0}, xl1 = u32x4{0, 0, 0, 0};
  if (a.x != nullptr) {
    xl0 = ld16(a.x + orow * 128 + 32 * h + 8 * half);
    xl1 = ld16(a.x + orow * 128 + 32 * h + 16 + 8 * half);
  }
  u32x2 gr[4];
  runs(gl0, gl1, gr);
  // ---- og = O / l * sigmoid(g) -> LDS (the V rows of every wave are then dead) ----
  const float inv = 1.0f / l;
  __syncthreads();
  uint16_t* og = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float v0 = o[4 * j] * inv * sigmoidf_(bflo(gr[j][0]));
    const float v1 = o[4 * j + 1] * inv * sigmoidf_(bfhi(gr[j][0]));
    const float v2 = o[4 * j + 2] * inv * sigmoidf_(bflo(gr[j][1]));
    const float v3 = o[4 * j + 3] * inv * sigmoidf_(bfhi(gr[j][1]));
    *reinterpret_cast<u32x2*>(og + li * kWinOgPitch + 32 * h + 8 * j + 4 * half) =
        u32x2{pack_bf2(v0, v1), pack_bf2(v2, v3)};
  }
  __syncthreads();
  // ---- out^T (channels 32 h .. + 31, this wave) = W_t2 og^T; * zgate + x ----
  f32x16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
  for (int kk = 0; kk < 8; ++kk)
    acc = mfma32(as_bf16x8(wr[kk]), as_bf16x8(ld16(og + li * kWinOgPitch + 16 * kk + 8 * half)), acc);
  u32x2 zg[4], xr[4];
  runs(zl0, zl1, zg);
  runs(xl0, xl1, xr);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float v[4] = {acc[4 * j] * bflo(zg[j][0]), acc[4 * j + 1] * bfhi(zg[j][0]),
                  acc[4 * j + 2] * bflo(zg[j][1]), acc[4 * j + 3] * bfhi(zg[j][1])};
    if (a.x != nullptr) {                                   // uniform
      v[0] += bflo(xr[j][0]); v[1] += bfhi(xr[j][0]); v[2] += bflo(xr[j][1]); v[3] += bfhi(xr[j][1]);
    }
    *reinterpret_cast<u32x2*>(a.out + orow * 128 + 32 * h + 8 * j + 4 * half) =
        u32x2{pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3])};
  }
}

// The per-atom plan: AdaLN of every atom for both sides from the given terms, q/g and k/v
// projected once per atom, the attention gathering each window's K / V rows, AdaLN-zero output.
int cross_prepared_run(const sf_cross_attention_args* a, Arena ws, hipStream_t st) {
  const int C = a->C, HD = a->H * a->D;
  const int64_t A = (int64_t)a->U * a->Qw, rows = (int64_t)a->S * A;
  int rc;
  void* hq = ws.take((size_t)rows * C * 2);
  void* hk = ws.take((size_t)rows * C * 2);
  void* yq = ws.take((size_t)rows * 2 * HD * 2);
  void* ykv = ws.take((size_t)a->S * (A + 1) * 2 * HD * 2);
  void* o = ws.take((size_t)rows * HD * 2);
  if (C == 128 && 2 * HD == 256) {                   // LN + both projections in one pass
    Adaln2Args f{};
    f.rows = rows; f.A = A; f.S = a->S; f.blocks = (int)((rows + 31) / 32);
    f.x = static_cast<const uint16_t*>(a->xq);
    f.q_scale = static_cast<const uint16_t*>(a->pre_q_scale); f.q_shift = static_cast<const uint16_t*>(a->pre_q_shift);
    f.k_scale = static_cast<const uint16_t*>(a->pre_k_scale); f.k_shift = static_cast<const uint16_t*>(a->pre_k_shift);
    f.prs = a->pre_rs;
    f.wqg = static_cast<const uint16_t*>(a->w_qg); f.wkv = static_cast<const uint16_t*>(a->w_kv); f.bqg = a->b_qg;
    f.yq = static_cast<uint16_t*>(yq); f.ykv = static_cast<uint16_t*>(ykv);
    // two workgroups per worker (one per side), workers a multiple of 8: the resident workgroups
    // or enough for every block, whichever is fewer
    const int resident = sf_resident_workgroups(reinterpret_cast<const void*>(adaln2_proj_kernel), 512);
    const int workers = std::max(8, std::min(resident / 2, (f.blocks + 7) / 8 * 8) / 8 * 8);
    hipLaunchKernelGGL(adaln2_proj_kernel, dim3(2 * workers), dim3(512), 0, st, f);
    if ((rc = sf_check_launch("adaln2_proj_kernel"))) return rc;
  } else {
  for (int side = 0; side < 2; ++side) {
    sf_layer_norm_args ln{};
    ln.M = rows; ln.C = C; ln.eps = 1e-5f;
    ln.x = a->xq; ln.x_rs = C; ln.y = side ? hk : hq; ln.y_rs = C;
    ln.scale = side ? a->pre_k_scale : a->pre_q_scale; ln.shift = side ? a->pre_k_shift : a->pre_q_shift;
    ln.cond_rows = A; ln.cond_rs = a->pre_rs;
    if ((rc = sf_hip_layer_norm_fwd(&ln, st))) return rc;
  }
  sf_linear_args p{};
  p.M = rows; p.N = 2 * HD; p.K = C; p.x = hq; p.x_rs = C; p.wt = a->w_qg; p.bias = a->b_qg;
  p.mul_rows = 1; p.y = yq; p.y_rs = 2 * HD;
  if ((rc = sf_hip_linear_fwd(&p, st))) return rc;
  sf_linear_args pk{};                       // per sample: rows 0..A-1 of its [A + 1] block
  pk.M = A; pk.N = 2 * HD; pk.K = C; pk.x = hk; pk.x_rs = C; pk.wt = a->w_kv; pk.mul_rows = 1;
  pk.y = ykv; pk.y_rs = 2 * HD; pk.batch = a->S; pk.x_bs = A * C; pk.y_bs = (A + 1) * 2 * HD;
  if ((rc = sf_hip_linear_fwd(&pk, st))) return rc;
  const int words = 2 * HD * 2 / 16;
  hipLaunchKernelGGL(zero_rows_kernel, dim3((unsigned)((a->S * words + 255) / 256)), dim3(256), 0, st,
                     reinterpret_cast<u32x4*>(static_cast<uint16_t*>(ykv) + A * 2 * HD), (A + 1) * 2 * HD * 2 / 16,
                     a->S, words);
  if ((rc = sf_check_launch("zero_rows_kernel"))) return rc;
  }
  if (a->Qw == 32 && a->Kw == 128 && a->H == 4 && a->D == 32 && C == 128 && (int64_t)a->S * a->U < (1ll << 31)) {
    WinFusedArgs f{};
    f.S = a->S; f.U = a->U; f.A = (int)A;
    f.yq = static_cast<const uint16_t*>(yq); f.ykv = static_cast<const uint16_t*>(ykv);
    f.gidx = a->gather_idx; f.gmask = a->gather_mask; f.mask_q = a->mask_q; f.mask_k = a->mask_k;
    f.bias = static_cast<const uint16_t*>(a->bias); f.w_t2 = static_cast<const uint16_t*>(a->w_t2);
    f.zgate = static_cast<const uint16_t*>(a->pre_zgate); f.zrs = a->pre_rs;
    f.x = a->add_residual ? static_cast<const uint16_t*>(a->xq) : nullptr;
    f.out = static_cast<uint16_t*>(a->out);
    const float scale = a->scale > 0.f ? a->scale : 1.0f / std::sqrt((float)a->D);
    f.scale = scale;
    hipLaunchKernelGGL(window_attn_out_kernel, dim3((unsigned)(a->S * a->U)), dim3(256), 0, st, f);
    return sf_check_launch("window_attn_out_kernel");
  }
  const sf_attention_args t = cross_prepared_attn_args(a, yq, ykv, o);
  const size_t split = sf_attention_workspace_bytes(&t);
  void* split_ws = ws.take(split);
  if ((rc = sf_attention_run(&t, split_ws, split, st))) return rc;
  return zero_init_out(rows, C, HD, o, nullptr, A, C, nullptr, nullptr, a->w_t2, a->add_residual ? a->xq : nullptr,
                       a->out, ws, st, a->pre_zgate, a->pre_rs);
}
}  // namespace

extern "C" int sf_hip_cross_attention_fwd(const sf_cross_attention_args* a, void* workspace,
                                          size_t workspace_bytes, void* stream) {
  if (a != nullptr && cross_prepared(a)) {
    if (a->xq == nullptr || a->out == nullptr || a->w_qg == nullptr || a->w_kv == nullptr || a->w_t2 == nullptr ||
        a->gather_mask == nullptr || a->pre_q_shift == nullptr || a->pre_k_scale == nullptr ||
        a->pre_k_shift == nullptr || a->pre_zgate == nullptr) {
      sf_set_error("cross_attention: the per-atom plan needs xq, out, w_qg, w_kv, w_t2, gather_mask and all five "
                   "pre_* terms");
      return 1;
    }
    if (a->S <= 0 || a->U <= 0 || a->Qw <= 0 || a->Kw <= 0 || a->C <= 0 || a->H <= 0 || a->D <= 0 ||
        a->pre_rs < a->C || (2 * a->H * a->D) % 8 != 0) {
      sf_set_error("cross_attention: sizes must be positive, pre_rs >= C and 2HD a multiple of 8"); return 1;
    }
    if (workspace == nullptr || workspace_bytes < cross_ws(a)) {
      sf_set_error("cross_attention: workspace of %zu bytes needed, %zu given", cross_ws(a), workspace_bytes);
      return 1;
    }
    return cross_prepared_run(a, Arena{static_cast<char*>(workspace)}, reinterpret_cast<hipStream_t>(stream));
  }
  if (a == nullptr || a->xq == nullptr || a->out == nullptr || a->w_qg == nullptr || a->w_kv == nullptr ||
      a->w_t2 == nullptr || a->w_zc == nullptr || a->cond_q == nullptr || a->cond_k == nullptr) {
    sf_set_error("cross_attention: xq, out, weights and both conditions must be non-null"); return 1;
  }
  if ((a->gather_idx == nullptr) == (a->xk == nullptr) || (a->gather_idx && a->gather_mask == nullptr)) {
    sf_set_error("cross_attention: give either xk or gather_idx + gather_mask"); return 1;
  }
  if (a->S <= 0 || a->U <= 0 || a->Qw <= 0 || a->Kw <= 0 || a->C <= 0 || a->H <= 0 || a->D <= 0) {
    sf_set_error("cross_attention: sizes must be positive"); return 1;
  }
  if (workspace == nullptr || workspace_bytes < cross_ws(a)) {
    sf_set_error("cross_attention: workspace of %zu bytes needed, %zu given", cross_ws(a), workspace_bytes);
    return 1;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  Arena ws{static_cast<char*>(workspace)};
  const int C = a->C, HD = a->H * a->D;
  const int64_t qrows = (int64_t)a->S * a->U * a->Qw, krows = (int64_t)a->S * a->U * a->Kw;
  int rc;
  // gathered keys are never materialised: their LayerNorm reads the query rows through the gather
  const void* xk = a->gather_idx ? a->xq : a->xk;
  // the two AdaLN chains take their scratch first, in the order cross_ws counts it
  Arena side_q = ws;
  Arena side_k = ws;
  for (int i = 0; i < 3; ++i) side_k.take((size_t)a->U * a->Qw * C * 2);
  Arena rest = side_k;
  for (int i = 0; i < 3; ++i) rest.take((size_t)a->U * a->Kw * C * 2);
  void* hq = rest.take((size_t)qrows * C * 2);
  void* hk = rest.take((size_t)krows * C * 2);
  if ((rc = adaln(qrows, C, a->xq, a->cond_q, (int64_t)a->U * a->Qw, C, nullptr, nullptr, a->lnc_w_q, a->lnc_b_q,
                  a->w_scale_q, a->b_scale_q, a->w_shift_q, side_q, hq, st)))
    return rc;
  if ((rc = adaln(krows, C, xk, a->cond_k, (int64_t)a->U * a->Kw, C, nullptr, nullptr, a->lnc_w_k, a->lnc_b_k,
                  a->w_scale_k, a->b_scale_k, a->w_shift_k, side_k, hk, st, a->gather_idx, a->gather_mask,
                  (int64_t)a->U * a->Kw, (int64_t)a->U * a->Qw)))
    return rc;
  void* yq = rest.take((size_t)qrows * 2 * HD * 2);
  void* yk = rest.take((size_t)krows * 2 * HD * 2);
  void* o = rest.take((size_t)qrows * HD * 2);
  sf_linear_args p{};
  p.M = qrows; p.N = 2 * HD; p.K = C; p.x = hq; p.x_rs = C; p.wt = a->w_qg; p.bias = a->b_qg;
  p.mul_rows = 1; p.y = yq; p.y_rs = 2 * HD;
  if ((rc = sf_hip_linear_fwd(&p, st))) return rc;
  p.M = krows; p.x = hk; p.wt = a->w_kv; p.bias = nullptr; p.y = yk;
  if ((rc = sf_hip_linear_fwd(&p, st))) return rc;
  const sf_attention_args t = cross_attn_args(a, yq, yk, o);
  const size_t split = sf_attention_workspace_bytes(&t);
  void* split_ws = rest.take(split);
  if ((rc = sf_attention_run(&t, split_ws, split, st))) return rc;
  return zero_init_out(qrows, C, HD, o, a->cond_q, (int64_t)a->U * a->Qw, C, a->w_zc, a->b_zc, a->w_t2,
                       a->add_residual ? a->xq : nullptr, a->out, rest, st);
}

namespace {

size_t transition_ws(const sf_transition_args* a) {
  Arena ws{nullptr};
  const int64_t rows = (int64_t)a->S * a->N;
  const bool cond_gemms = a->cond && !a->pre_scale;
  if (cond_gemms) {                          // LN(cond), scale, shift, zgate
    ws.take((size_t)a->N * a->Cs * 2); ws.take((size_t)a->N * a->C * 2); ws.take((size_t)a->N * a->C * 2);
    ws.take((size_t)a->N * a->C * 2);
  }
  ws.take((size_t)rows * a->C * 2);          // h
  ws.take((size_t)rows * a->I * 2);          // gated intermediate
  if (cond_gemms) ws.take((size_t)a->N * a->C * 2);
  return ws.off;
}

}  // namespace

extern "C" size_t sf_hip_transition_workspace_bytes(const sf_transition_args* a) {
  return a == nullptr ? 0 : transition_ws(a);
}

extern "C" int sf_hip_transition_fwd(const sf_transition_args* a, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  if (a == nullptr || a->x == nullptr || a->out == nullptr || a->w1 == nullptr || a->w2 == nullptr) {
    sf_set_error("transition: x, out, w1 and w2 must be non-null"); return 1;
  }
  if (a->S <= 0 || a->N <= 0 || a->C <= 0 || a->I <= 0 || a->C % 64 != 0 || a->I % 4 != 0 ||
      (a->cond && !a->pre_scale && a->Cs <= 0)) {
    sf_set_error("transition: need positive sizes, C %% 64 == 0 and I %% 4 == 0 (S=%d N=%d C=%d I=%d Cs=%d)",
                 a->S, a->N, a->C, a->I, a->Cs);
    return 1;
  }
  const bool pre = a->pre_scale != nullptr;
  if (pre && (a->pre_shift == nullptr || a->pre_zgate == nullptr || a->pre_rs < a->C)) {
    sf_set_error("transition: pre_scale needs pre_shift, pre_zgate and pre_rs >= C"); return 1;
  }
  if (!pre && a->cond && (a->w_scale == nullptr || a->w_shift == nullptr || a->w_zc == nullptr)) {
    sf_set_error("transition: a condition needs w_scale, w_shift and w_zc"); return 1;
  }
  if (workspace == nullptr || workspace_bytes < transition_ws(a)) {
    sf_set_error("transition: workspace of %zu bytes needed, %zu given", transition_ws(a), workspace_bytes);
    return 1;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  Arena ws{static_cast<char*>(workspace)};
  const int64_t rows = (int64_t)a->S * a->N;
  int rc;
  void* h = nullptr;
  void *c_scale = nullptr, *c_shift = nullptr, *c_zgate = nullptr;
  const bool fused_cond = a->cond && !pre && cond_terms_ok(a->C, a->Cs, a->cond, a->w_scale, a->w_shift, a->w_zc);
  {
    Arena probe = ws;                        // the AdaLN scratch first, as in transition_ws
    if (a->cond && !pre) {
      probe.take((size_t)a->N * a->Cs * 2);
      c_scale = probe.take((size_t)a->N * a->C * 2); c_shift = probe.take((size_t)a->N * a->C * 2);
      c_zgate = probe.take((size_t)a->N * a->C * 2);
    }
    h = probe.take((size_t)rows * a->C * 2);
    if (pre || fused_cond) {
      // the conditioning terms of this layer in one launch (or given), then the modulated LayerNorm
      if (fused_cond && (rc = cond_terms(a->N, a->C, a->Cs, a->cond, a->lnc_w, a->lnc_b, a->w_scale, a->b_scale,
                                         a->w_shift, a->w_zc, a->b_zc, c_scale, c_shift, c_zgate, st))) {
        return rc;
      }
      sf_layer_norm_args ln{};
      ln.M = rows; ln.C = a->C; ln.eps = 1e-5f;
      ln.x = a->x; ln.x_rs = a->C; ln.y = h; ln.y_rs = a->C;
      ln.scale = pre ? a->pre_scale : c_scale; ln.shift = pre ? a->pre_shift : c_shift; ln.cond_rows = a->N;
      ln.cond_rs = pre ? a->pre_rs : a->C;
      if ((rc = sf_hip_layer_norm_fwd(&ln, st))) return rc;
    } else if ((rc = adaln(rows, a->C, a->x, a->cond, a->N, a->Cs, a->ln_w, a->ln_b, a->lnc_w, a->lnc_b,
                           a->w_scale, a->b_scale, a->w_shift, ws, h, st))) {
      return rc;
    }
    ws = probe;
  }
  void* c = ws.take((size_t)rows * a->I * 2);
  sf_linear_args g{};
  g.M = rows; g.N = 2 * a->I; g.K = a->C; g.x = h; g.x_rs = a->C; g.wt = a->w1; g.mul_rows = 1;
  g.y = c; g.y_rs = a->I; g.glu = 1;
  if ((rc = sf_hip_linear_fwd(&g, st))) return rc;
  return zero_init_out(rows, a->C, a->I, c, pre || fused_cond ? nullptr : a->cond, a->N, a->Cs, a->w_zc, a->b_zc,
                       a->w2, a->add_residual ? a->x : nullptr, a->out, ws, st,
                       pre ? a->pre_zgate : c_zgate, pre ? a->pre_rs : a->C);
}

namespace {

// W'[j, k] = W[j, k] * g[j / C, k] for the scale and shift weights (blockIdx.y picks which),
// eight bf16 per thread; Cs % 8 == 0 keeps each group of eight inside one row.
__global__ void __launch_bounds__(256) fold_gamma_kernel(const uint16_t* __restrict__ w0,
                                                         const uint16_t* __restrict__ w1,
                                                         const float* __restrict__ g, uint16_t* o0,
                                                         uint16_t* o1, int64_t groups, int C, int Cs) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= groups) return;
  const uint16_t* w = blockIdx.y ? w1 : w0;
  uint16_t* o = blockIdx.y ? o1 : o0;
  const int64_t e = i * 8;
  const int64_t row = e / Cs;
  const int k0 = (int)(e - row * Cs);
  const float* gl = g + (row / C) * Cs + k0;
  const u32x4 v = ld16(w + e);
  u32x4 r;
  r[0] = pack_bf2(bflo(v[0]) * gl[0], bfhi(v[0]) * gl[1]);
  r[1] = pack_bf2(bflo(v[1]) * gl[2], bfhi(v[1]) * gl[3]);
  r[2] = pack_bf2(bflo(v[2]) * gl[4], bfhi(v[2]) * gl[5]);
  r[3] = pack_bf2(bflo(v[3]) * gl[6], bfhi(v[3]) * gl[7]);
  st16(o + e, r);
}

size_t conditioning_ws(const sf_diffusion_conditioning_args* a) {
  Arena ws{nullptr};
  ws.take((size_t)a->rows * a->Cs * 2);                  // LN(c)
  ws.take((size_t)a->L * a->C * a->Cs * 2);              // W_scale * g
  ws.take((size_t)a->L * a->C * a->Cs * 2);              // W_shift * g
  return ws.off;
}

}  // namespace

extern "C" size_t sf_hip_diffusion_conditioning_workspace_bytes(const sf_diffusion_conditioning_args* a) {
  return a == nullptr ? 0 : conditioning_ws(a);
}

extern "C" int sf_hip_diffusion_conditioning_fwd(const sf_diffusion_conditioning_args* a, void* workspace,
                                                 size_t workspace_bytes, void* stream) {
  if (a == nullptr || a->cond == nullptr || a->lnc_w == nullptr || a->w_scale == nullptr ||
      a->w_shift == nullptr || a->w_zc == nullptr || a->scale == nullptr || a->shift == nullptr ||
      a->zgate == nullptr) {
    sf_set_error("diffusion_conditioning: cond, lnc_w, the three weights and the three outputs must be non-null");
    return 1;
  }
  if (a->rows < 0 || a->L <= 0 || a->C <= 0 || a->Cs <= 0 || a->Cs % 8 != 0 || a->Cs > 2048) {
    sf_set_error("diffusion_conditioning: need rows >= 0, L, C > 0 and 0 < Cs <= 2048 with Cs %% 8 == 0 "
                 "(rows=%lld L=%d C=%d Cs=%d)", (long long)a->rows, a->L, a->C, a->Cs);
    return 1;
  }
  const int64_t LC = (int64_t)a->L * a->C;
  if (LC > 0x7fffffff || a->out_rs < LC) {
    sf_set_error("diffusion_conditioning: need L*C < 2^31 and out_rs >= L*C (L*C=%lld out_rs=%lld)",
                 (long long)LC, (long long)a->out_rs);
    return 1;
  }
  if (workspace == nullptr || workspace_bytes < conditioning_ws(a)) {
    sf_set_error("diffusion_conditioning: workspace of %zu bytes needed, %zu given", conditioning_ws(a),
                 workspace_bytes);
    return 1;
  }
  if (((reinterpret_cast<uintptr_t>(a->w_scale) | reinterpret_cast<uintptr_t>(a->w_shift)) & 15) != 0) {
    sf_set_error("diffusion_conditioning: w_scale and w_shift must be 16-byte aligned");
    return 1;
  }
  if (a->rows == 0) return 0;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  Arena ws{static_cast<char*>(workspace)};
  void* cn = ws.take((size_t)a->rows * a->Cs * 2);
  void* ws_scale = ws.take((size_t)LC * a->Cs * 2);
  void* ws_shift = ws.take((size_t)LC * a->Cs * 2);
  sf_layer_norm_args ln{};
  ln.M = a->rows; ln.C = a->Cs; ln.eps = 1e-5f;
  ln.x = a->cond; ln.x_rs = a->Cs; ln.y = cn; ln.y_rs = a->Cs;
  int rc = sf_hip_layer_norm_fwd(&ln, st);
  if (rc) return rc;
  const int64_t groups = LC * a->Cs / 8;
  hipLaunchKernelGGL(fold_gamma_kernel, dim3((unsigned)((groups + 255) / 256), 2), dim3(256), 0, st,
                     static_cast<const uint16_t*>(a->w_scale), static_cast<const uint16_t*>(a->w_shift),
                     a->lnc_w, static_cast<uint16_t*>(ws_scale), static_cast<uint16_t*>(ws_shift), groups,
                     a->C, a->Cs);
  if ((rc = sf_check_launch("fold_gamma_kernel"))) return rc;
  sf_linear_args l{};
  l.M = a->rows; l.N = (int32_t)LC; l.K = a->Cs; l.x = cn; l.x_rs = a->Cs; l.mul_rows = 1;
  l.wt = ws_scale; l.bias = a->b_scale; l.post_sigmoid = 1; l.y = a->scale; l.y_rs = a->out_rs;
  if ((rc = sf_hip_linear_fwd(&l, st))) return rc;
  l.wt = ws_shift; l.bias = nullptr; l.post_sigmoid = 0; l.y = a->shift;
  if ((rc = sf_hip_linear_fwd(&l, st))) return rc;
  l.x = a->cond; l.wt = a->w_zc; l.bias = a->b_zc; l.post_sigmoid = 1; l.y = a->zgate;
  return sf_hip_linear_fwd(&l, st);
}
