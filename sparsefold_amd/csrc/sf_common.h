// Shared device helpers for the gfx950 (CDNA4) kernels: bf16 packing, 16-byte vector
// loads, MFMA wrappers and wave-level reductions.  Written for wave64.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/sparsefold_hip.h"

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(2))) float f32x2;

#define SF_LOG2E 1.4426950408889634f
// Logit (log2 domain) of a masked key.  Finite, so a query whose keys are all masked
// sees identical logits and weighs every key equally -- the reference's -finfo.max rule.
// -2^99: exact in bf16 and fp32, and any |q.k| logit is absorbed when added to it.
#define SF_MASKED_LOGIT (-6.338253001141147e29f)

__device__ __forceinline__ float bf2f(uint16_t u) { return __uint_as_float((uint32_t)u << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) {
  __bf16 b = (__bf16)f;  // v_cvt_pk_bf16_f32: round to nearest even
  return __builtin_bit_cast(uint16_t, b);
}
__device__ __forceinline__ float bflo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bfhi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  return (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
}

// Two floats -> packed bf16 pair (one v_cvt_pk_bf16_f32, round to nearest even).
__device__ __forceinline__ bf16x2 cvt_bf2(float lo, float hi) {
  return __builtin_convertvector(f32x2{lo, hi}, bf16x2);
}
// acc + lo + hi of a packed bf16 pair, fp32 accumulation (v_dot2c_f32_bf16 against ones).
__device__ __forceinline__ float add_bf2(bf16x2 v, float acc) {
  const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(v, one, acc, false);
}

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
// Non-temporal (streaming) 16-byte store: for outputs that a later kernel reads, written in runs
// of whole 128-byte lines by each instruction.  Scattered partial-line streams are slower than
// plain stores (measured 3x on 8-byte scattered stores), so use it only for full-line runs.
__device__ __forceinline__ void st16_stream(void* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// D(32x32) += A(32x16) * B(16x32), bf16 inputs, fp32 accumulation.
// Lane l: A row l%32 / B column l%32, k = 8*(l/32) .. +7; D row 8*(r/4)+4*(l/32)+r%4, col l%32.
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
// Logistic sigmoid from exp2: 1 / (1 + 2^(-x log2 e)).
__device__ __forceinline__ float sigmoidf_(float x) { return fast_rcp(1.0f + fast_exp2(-x * SF_LOG2E)); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Load 8 bf16 starting at element `d0` of a row with `n` valid elements; elements past n
// read as 0.  `vec` selects the 16-byte path (caller guarantees alignment and n % 8 == 0).
__device__ __forceinline__ u32x4 load8_guard(const uint16_t* row, int d0, int n, bool vec) {
  if (vec) {
    if (d0 < n) return ld16(row + d0);
    return u32x4{0, 0, 0, 0};
  }
  uint32_t w[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    uint32_t lo = (d0 + 2 * e < n) ? row[d0 + 2 * e] : 0;
    uint32_t hi = (d0 + 2 * e + 1 < n) ? row[d0 + 2 * e + 1] : 0;
    w[e] = lo | (hi << 16);
  }
  return u32x4{w[0], w[1], w[2], w[3]};
}

// LayerNorm (eps 1e-5, no affine: gamma / beta are folded into the consuming weight) of 32
// positions x 16*NC channels, straight into MFMA operand registers: lane (li, half)
// holds channels 16*kk + 8*half .. +7 of position li for kk = 0..NC-1 -- the same registers
// serve as A operand (rows = positions) and as B operand (columns = positions).
template <int NC>
__device__ __forceinline__ void ln_operands(const u32x4 (&x)[NC], bool valid, bf16x8 (&xo)[NC]) {
  constexpr float kInvC = 1.0f / (16 * NC);
  float sum = 0.f;
#pragma unroll
  for (int kk = 0; kk < NC; ++kk)
#pragma unroll
    for (int e = 0; e < 4; ++e) sum += bflo(x[kk][e]) + bfhi(x[kk][e]);
  sum += __shfl_xor(sum, 32);
  const float mean = sum * kInvC;
  float sq = 0.f;
#pragma unroll
  for (int kk = 0; kk < NC; ++kk)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float d0 = bflo(x[kk][e]) - mean, d1 = bfhi(x[kk][e]) - mean;
      sq += d0 * d0 + d1 * d1;
    }
  sq += __shfl_xor(sq, 32);
  const float rstd = valid ? rsqrtf(sq * kInvC + 1e-5f) : 0.f;
#pragma unroll
  for (int kk = 0; kk < NC; ++kk)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bf16x2 v = cvt_bf2((bflo(x[kk][e]) - mean) * rstd, (bfhi(x[kk][e]) - mean) * rstd);
      xo[kk][2 * e] = v[0];
      xo[kk][2 * e + 1] = v[1];
    }
}
__device__ __forceinline__ void ln128_operands(const u32x4 (&x)[8], bool valid, bf16x8 (&xo)[8]) {
  ln_operands<8>(x, valid, xo);
}

// LDS barrier that leaves global loads and stores in flight: this wave's LDS accesses complete
// (lgkmcnt 0; vmcnt / expcnt left at their maxima), then the workgroup barrier.  __syncthreads()
// also waits for every global access of the wave (vmcnt 0), stores included.
__device__ __forceinline__ void lds_only_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Thread-local last-error plumbing shared by all C entry points.
void sf_set_error(const char* fmt, ...);
int sf_check_launch(const char* what);

// Workgroups of `kernel` (launched with `threads` threads, no dynamic LDS) that the current
// device holds at once: CUs x occupancy; cached per (device, kernel).  At least 1.
int sf_resident_workgroups(const void* kernel, int threads);

// Attention with an optional workspace (library-internal; the C entry point has none): with a
// workspace of sf_attention_workspace_bytes, per-wave tasks on a grid too small for the GPU
// split their key range into slices merged by a combine kernel.
size_t sf_attention_workspace_bytes(const sf_attention_args* a);
int sf_attention_run(const sf_attention_args* a, void* workspace, size_t workspace_bytes, hipStream_t stream);
// Shared-bias attention (5 samples, head dim 48, one bias for every sample): whether it serves
// `a` (else *why names the first condition that fails), and its launch.
bool sf_sb_attention_ok(const sf_attention_args* a, const char** why);
int sf_sb_attention_launch(const sf_attention_args* a, hipStream_t stream);
