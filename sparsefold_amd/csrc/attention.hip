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

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7) == 0; }

}  // namespace

extern "C" int sf_hip_attention_fwd(const sf_attention_args* a, void* stream) {
  if (a == nullptr) { sf_set_error("attention: null args"); return 1; }
  if (a->q == nullptr || a->k == nullptr || a->v == nullptr || a->out == nullptr) {
    sf_set_error("attention: q, k, v and out must be non-null"); return 1;
  }
  if (a->B0 <= 0 || a->B1 <= 0 || a->Q <= 0 || a->K <= 0 || a->H <= 0 || a->D <= 0 || a->Dv <= 0) {
    sf_set_error("attention: sizes must be positive (B0=%d B1=%d Q=%d K=%d H=%d D=%d Dv=%d)",
                 a->B0, a->B1, a->Q, a->K, a->H, a->D, a->Dv);
    return 1;
  }
  const int dmax = a->D > a->Dv ? a->D : a->Dv;
  if (dmax > 64) { sf_set_error("attention: head dims above 64 are not supported (D=%d Dv=%d)", a->D, a->Dv); return 1; }
  if ((int64_t)a->B0 * a->B1 > 65535 || a->H > 65535) {
    sf_set_error("attention: batch (%d) or heads (%d) exceed the grid limit", a->B0 * a->B1, a->H); return 1;
  }
  // 16-byte path for q/k/v rows: head dims multiple of 8, row/head strides multiple of 8,
  // 16-byte aligned bases.
  bool vec = (a->D % 8 == 0) && (a->Dv % 8 == 0) && aligned16(a->q) && aligned16(a->k) && aligned16(a->v);
  for (int s = 0; s < 4 && vec; ++s)
    vec = (a->q_s[s] % 8 == 0) && (a->k_s[s] % 8 == 0) && (a->v_s[s] % 8 == 0);
  bool vec_out = aligned8(a->out);
  for (int s = 0; s < 4 && vec_out; ++s) vec_out = (a->o_s[s] % 4 == 0);
  dim3 grid((a->Q + kQB - 1) / kQB, a->H, a->B0 * a->B1);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (dmax <= 32)
    hipLaunchKernelGGL(attention_fwd_kernel<32>, grid, dim3(256), 0, st, *a, (int)vec, (int)vec_out);
  else
    hipLaunchKernelGGL(attention_fwd_kernel<64>, grid, dim3(256), 0, st, *a, (int)vec, (int)vec_out);
  return sf_check_launch("attention_fwd_kernel");
}
