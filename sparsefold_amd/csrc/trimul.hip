// Triangle multiplicative update, outgoing ("...ikc,...jkc->...ijc") and incoming
// ("...kjc,...kic->...ijc") edges: TriangleMultiplication.forward (blocks.py:486-566), C = 128.
//
//   1. trimul_proj_kernel   x = LN(z) (left_norm_input) straight into MFMA operands; the gated
//                           linear unit sigmoid(x W_g) * (x W_p) (primitives.py:586-631) for the
//                           2C projected channels, zero where mask[i] & mask[k] is false
//                           (blocks.py:516-530), written channel-major into zero-padded planes
//                           [c][Pn][Pn] (Pn = N rounded up to 64): a = channel 2c, b = 2c + 1
//                           ("(c i2) b n -> i2 c b n", :540).  Outgoing edges store position
//                           (i, k) at row i, column k; incoming edges walk z column-wise and store
//                           position (k, j) at row j, column k -- the transposed planes -- so that
//                           both edges contract over the planes' contiguous dimension.
//   2. per-channel product  t[c][i][j] = sum_k A[c][i][k] B[c][j][k] (blocks.py:555): one batched
//                           NT GEMM over the 128 channels (sf_hip_linear_fwd, batched form) with
//                           (A, B) = (a, b) for outgoing and (b^T, a^T) for incoming edges; the zero
//                           padding of the contraction dimension adds nothing.
//   3. trimul_out_kernel    LN over the channels of t (center_norm, dim=-3), output projection,
//                           gate sigmoid(LN(z) W_gl) recomputed from z, out = z + update
//                           (blocks.py:561-566).
// LayerNorm affines are folded into the consuming weights: (LN0(x) g + b) W^T =
// LN0(x) (W * g)^T + W b.  trimul_fold_kernel writes the folded weights into the workspace.
#include <algorithm>
#include <mutex>

#include "sf_common.h"

namespace {

constexpr int kC = 128;            // channels (the pair representation's width)
constexpr int kWS = kC + 8;        // LDS row stride of a [rows][128] bf16 weight (bank padding)
constexpr int kTW = 8;             // waves per workgroup of both position kernels
constexpr int kGlu = 4 * kC;       // GLU rows: gate a, gate b, projection a, projection b
constexpr int kTP = 34;            // LDS pitch of a staged [128 channels][32 positions] product block
static_assert(kC * kTP == 32 * kWS, "the staged product block fills a wave's output rows exactly");

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }
int64_t plane_stride(int N) { return ((int64_t)N * N + 31) & ~(int64_t)31; }
int padded_n(int N) { return (N + 63) & ~63; }

// Folded weights and offsets, one block of rows each: GLU (left_norm), output (center_norm),
// gate (left_norm).
struct FoldArgs {
  const uint16_t* w[3];
  const float* g[3];
  const float* b[3];
  int rows[3];
  uint16_t* wf[3];
  float* off[3];
};

// one wave per weight row: lane l folds columns 2l, 2l + 1
__global__ __launch_bounds__(256) void trimul_fold_kernel(const FoldArgs a) {
  int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, c = 2 * lane;
  int s = 0;
  while (s < 3 && n >= a.rows[s]) n -= a.rows[s++];
  if (s >= 3) return;                                  // uniform over the wave
  const uint32_t raw = *reinterpret_cast<const uint32_t*>(a.w[s] + (int64_t)n * kC + c);
  const float v0 = bflo(raw), v1 = bfhi(raw);
  const float* g = a.g[s];
  const float* b = a.b[s];
  *reinterpret_cast<uint32_t*>(a.wf[s] + (int64_t)n * kC + c) = pack_bf2(g ? v0 * g[c] : v0, g ? v1 * g[c + 1] : v1);
  const float off = wave_sum(b ? v0 * b[c] + v1 * b[c + 1] : 0.f);
  if (lane == 0) a.off[s][n] = off;
}

struct ProjArgs {
  int N, Pn, incoming;           // Pn: padded plane side (multiple of 64)
  const uint16_t* z;             // [N*N, 128]
  const uint8_t* mask;           // [N] or NULL
  const uint16_t* w;             // folded GLU [512, 128]
  const float* off;              // [512]
  uint16_t* a;                   // [128][Pn][Pn]
  uint16_t* b;                   // [128][Pn][Pn]
  int items, items_per_wave;     // blocks of 32 plane columns: Pn rows x Pn / 32
};

// D^T = W X^T per 32 channels x 32 positions: lane (li, half) ends with position li (plane column
// 32 cb + li) at channels 32 nb + 8(r/4) + 4 half + r%4; each register is one 2-byte store, and
// the 32 lanes of a half write 64 contiguous bytes of one plane row.
// No wait covers a store: the next item's z rows and mask bytes are loaded before this item's
// products, unconditionally (positions past N read position 0; their values are replaced by
// zeros), and normalised after its stores.  With the loads predicated, the mask read between the
// stores and the normalisation at the top of the loop, every item waited for the previous item's
// stores.
__global__ __launch_bounds__(64 * kTW) void trimul_proj_kernel(const ProjArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t sW[kGlu * kWS];
  __shared__ float sOff[kGlu];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, li = lane & 31;
  constexpr int kStage = kGlu * (kC / 8) / (64 * kTW);
  u32x4 st[kStage];
#pragma unroll
  for (int u = 0; u < kStage; ++u) {
    const int t = tid + u * 64 * kTW;
    st[u] = ld16(a.w + (int64_t)(t >> 4) * kC + (t & 15) * 8);
  }
#pragma unroll
  for (int u = 0; u < kStage; ++u) {
    const int t = tid + u * 64 * kTW;
    st16(&sW[(t >> 4) * kWS + (t & 15) * 8], st[u]);
  }
  for (int n = tid; n < kGlu; n += 64 * kTW) sOff[n] = a.off[n];
  __syncthreads();
  const int cbs = a.Pn / 32;                            // column blocks per plane row
  const int64_t plane = (int64_t)a.Pn * a.Pn;
  // the workgroup's items are base .. base + kTW * items_per_wave - 1, wave w taking every kTW-th:
  // neighbouring column blocks, whose stores fill the two halves of each 128-byte plane line, are
  // written together (one wave walking consecutive items came back to a line too late for L2)
  const int base = blockIdx.x * kTW * a.items_per_wave;
  // item -> plane row R, columns 32 cb .. 32 cb + 31; this lane's column col.  Outgoing: z position
  // (R, col); incoming: (col, R), so that the planes hold a^T and b^T
  auto load_item = [&](int item, u32x4 (&zn)[8], bool& ok, int& R, int& col, int& m0, int& m1) __attribute__((always_inline)) {
    R = item / cbs;
    col = 32 * (item - R * cbs) + li;
    const int za = a.incoming ? col : R, zb = a.incoming ? R : col;
    ok = za < a.N && zb < a.N;
    const uint16_t* zp = a.z + (ok ? (int64_t)za * a.N + zb : 0) * kC + 8 * half;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) zn[kk] = ld16(zp + 16 * kk);
    m0 = a.mask == nullptr ? 1 : a.mask[ok ? za : 0];
    m1 = a.mask == nullptr ? 1 : a.mask[ok ? zb : 0];
  };
  int item = base + wave;
  if (item >= a.items) return;                        // uniform: no barrier follows
  u32x4 zn[8];
  bool ok;
  int R, col, m0, m1;
  load_item(item, zn, ok, R, col, m0, m1);
  bf16x8 xo[8];
  ln128_operands(zn, ok, xo);
  bool keep = ok && m0 != 0 && m1 != 0;
  for (int k = 0;; ++k) {
    asm volatile("" ::: "memory");                    // the LDS weights are re-read every item
    const int nitem = item + kTW;
    const bool more = k + 1 < a.items_per_wave && nitem < a.items;   // uniform
    bool okn = false;
    int Rn = 0, coln = 0, m0n = 0, m1n = 0;
    if (more) load_item(nitem, zn, okn, Rn, coln, m0n, m1n);
    // store address = a uniform base per channel (scalar registers, recomputed every item from an
    // opaque plane stride; hoisted, the 16 channel offsets of each block took 32 VGPRs) plus this
    // lane's byte offset (half 4 planes in, plus the position; 64-bit: four planes pass 4 GiB
    // from N ~ 16k)
    int64_t pstride = plane;
    asm volatile("" : "+s"(pstride));
    const int64_t lofs = (4 * half * pstride + (int64_t)R * a.Pn + col) * 2;
#pragma unroll
    for (int side = 0; side < 2; ++side) {              // 0: a (even channels), 1: b (odd)
      char* dstp = reinterpret_cast<char*>(side ? a.b : a.a);
#pragma unroll
      for (int nb = 0; nb < kC / 32; ++nb) {
        const int rg = side * kC + 32 * nb + li;        // gate row of this lane's channel
        const int rp = 2 * kC + rg;                     // projection row
        f32x16 ag, ap;
#pragma unroll
        for (int e = 0; e < 16; ++e) { ag[e] = 0.f; ap[e] = 0.f; }
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          ag = mfma32(as_bf16x8(ld16(&sW[rg * kWS + 16 * kk + 8 * half])), xo[kk], ag);
          ap = mfma32(as_bf16x8(ld16(&sW[rp * kWS + 16 * kk + 8 * half])), xo[kk], ap);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int ch = 32 * nb + 8 * (r >> 2) + 4 * half + (r & 3);   // this register's channel
          const float v = sigmoidf_(ag[r] + sOff[side * kC + ch]) * (ap[r] + sOff[2 * kC + side * kC + ch]);
          char* cbase = dstp + (int64_t)(32 * nb + 8 * (r >> 2) + (r & 3)) * pstride * 2;   // uniform
          *reinterpret_cast<uint16_t*>(cbase + lofs) = f2bf(keep ? v : 0.f);
        }
      }
    }
    if (!more) break;
    ln128_operands(zn, okn, xo);                      // the next item, after this item's stores
    asm volatile("" : "+v"(m0n), "+v"(m1n));           // (its mask test stays here as well)
    keep = okn && m0n != 0 && m1n != 0;
    item = nitem; R = Rn; col = coln;
  }
}

struct OutArgs {
  int64_t P, Pp;
  const uint16_t* t;             // [128][Pp] channel-major product
  const uint16_t* z;             // [P, 128]
  const uint16_t* wo;            // folded output projection [128 out, 128 in]
  const float* oo;               // [128]
  const uint16_t* wg;            // folded gate [128 out, 128 in]
  const float* og;               // [128]
  int add_residual;
  uint16_t* out;                 // [P, 128]
  int items, items_per_wave;
};

// D^T = W X^T per 32 output channels x 32 positions: lane (li, half) ends with position li at
// channels 32 nb + 8(r/4) + 4 half + r%4; the gated update (plus the residual, taken from the z
// registers the gate's LayerNorm loaded) goes through a per-wave LDS row block so that every lane
// then writes whole 16-byte runs of the position-major output.
__global__ __launch_bounds__(64 * kTW) void trimul_out_kernel(const OutArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t sWo[kC * kWS];
  __shared__ __attribute__((aligned(16))) uint16_t sWg[kC * kWS];
  __shared__ float sOo[kC], sOg[kC];
  __shared__ __attribute__((aligned(16))) uint16_t sOut[kTW][32 * kWS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, li = lane & 31;
  constexpr int kStage = kC * (kC / 8) / (64 * kTW);
  u32x4 so_[kStage], sg_[kStage];
#pragma unroll
  for (int u = 0; u < kStage; ++u) {
    const int t = tid + u * 64 * kTW;
    so_[u] = ld16(a.wo + (int64_t)(t >> 4) * kC + (t & 15) * 8);
    sg_[u] = ld16(a.wg + (int64_t)(t >> 4) * kC + (t & 15) * 8);
  }
#pragma unroll
  for (int u = 0; u < kStage; ++u) {
    const int t = tid + u * 64 * kTW;
    st16(&sWo[(t >> 4) * kWS + (t & 15) * 8], so_[u]);
    st16(&sWg[(t >> 4) * kWS + (t & 15) * 8], sg_[u]);
  }
  for (int n = tid; n < kC; n += 64 * kTW) { sOo[n] = a.oo[n]; sOg[n] = a.og[n]; }
  __syncthreads();
  uint16_t* const rows = sOut[wave];
  // the workgroup's items are base .. base + kTW * items_per_wave - 1, wave w taking every kTW-th:
  // neighbouring blocks read the two 64-byte halves of each 128-byte line of t together (one wave
  // walking consecutive items came back to a line after L2 had dropped it: t was fetched twice)
  const int base = blockIdx.x * kTW * a.items_per_wave;
  for (int k = 0; k < a.items_per_wave; ++k) {
    const int item = base + k * kTW + wave;
    if (item >= a.items) break;
    const int64_t p = (int64_t)item * 32 + li;
    const bool ok = p < a.P;
    // the block's product, [128 channels][32 positions] (64 contiguous bytes per channel): 16-byte
    // loads into the wave's LDS rows at pitch 34, then each lane reads channels 16 kk + 8 half + 0..7
    // of its position.  Positions past P read the planes' padding (Pp >= item * 32 + 32).
    u32x4 tv[8], zn[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int q = lane + 64 * u, c = q >> 2, seg = q & 3;
      tv[u] = ld16(a.t + (int64_t)c * a.Pp + (int64_t)item * 32 + 8 * seg);
    }
    const uint16_t* zp = a.z + (ok ? p : 0) * kC + 8 * half;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) zn[kk] = ok ? ld16(zp + 16 * kk) : u32x4{0, 0, 0, 0};
    uint32_t* const rw = reinterpret_cast<uint32_t*>(rows);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int q = lane + 64 * u, c = q >> 2, seg = q & 3;
#pragma unroll
      for (int e = 0; e < 4; ++e) rw[(c * kTP + 8 * seg) / 2 + e] = tv[u][e];
    }
    asm volatile("" ::: "memory");                    // one wave's LDS accesses run in order
    u32x4 tn[8];
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t lo = rows[(16 * kk + 8 * half + 2 * e) * kTP + li];
        const uint32_t hi = rows[(16 * kk + 8 * half + 2 * e + 1) * kTP + li];
        w[e] = ok ? lo | (hi << 16) : 0u;
      }
      tn[kk] = u32x4{w[0], w[1], w[2], w[3]};
    }
    asm volatile("" ::: "memory");                    // (the rows are rewritten below)
    bf16x8 to[8], zo[8];
    ln128_operands(tn, ok, to);
    ln128_operands(zn, ok, zo);
#pragma unroll
    for (int nb = 0; nb < kC / 32; ++nb) {
      // residual z of this lane's update channels: channel 32 nb + 8 g + 4 half + e is word
      // 2 half + e/2 of zn[2 nb + g/2] in the lane of half g%2 -- this lane's own registers for
      // g%2 == half, the partner lane's (lane ^ 32) otherwise
      uint32_t zown[2][2], zrcv[2][2];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int w = 0; w < 2; ++w) {
          const u32x4 zw = zn[2 * nb + j];
          zown[j][w] = half ? zw[2 + w] : zw[w];
          zrcv[j][w] = (uint32_t)__shfl_xor((int)(half ? zw[w] : zw[2 + w]), 32);
        }
      f32x16 ao, ag;
#pragma unroll
      for (int e = 0; e < 16; ++e) { ao[e] = 0.f; ag[e] = 0.f; }
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        ao = mfma32(as_bf16x8(ld16(&sWo[(32 * nb + li) * kWS + 16 * kk + 8 * half])), to[kk], ao);
        ag = mfma32(as_bf16x8(ld16(&sWg[(32 * nb + li) * kWS + 16 * kk + 8 * half])), zo[kk], ag);
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c0 = 32 * nb + 8 * g + 4 * half;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = (ao[4 * g + e] + sOo[c0 + e]) * sigmoidf_(ag[4 * g + e] + sOg[c0 + e]);
        uint32_t u0 = pack_bf2(v[0], v[1]), u1 = pack_bf2(v[2], v[3]);   // the bf16 update
        if (a.add_residual) {                                            // out = update + z
          const bool mine = half == (g & 1);
          const uint32_t z0 = mine ? zown[g >> 1][0] : zrcv[g >> 1][0];
          const uint32_t z1 = mine ? zown[g >> 1][1] : zrcv[g >> 1][1];
          u0 = pack_bf2(bflo(u0) + bflo(z0), bfhi(u0) + bfhi(z0));
          u1 = pack_bf2(bflo(u1) + bflo(z1), bfhi(u1) + bfhi(z1));
        }
        *reinterpret_cast<u32x2*>(&rows[li * kWS + c0]) = u32x2{u0, u1};
      }
    }
    asm volatile("" ::: "memory");                    // one wave's LDS accesses run in order
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int q = lane + 64 * u, pos = q >> 4, c8 = (q & 15) * 8;
      const int64_t pp = (int64_t)item * 32 + pos;
      const u32x4 v = ld16(&rows[pos * kWS + c8]);
      if (pp < a.P) st16(a.out + pp * kC + c8, v);
    }
    asm volatile("" ::: "memory");                    // one wave's LDS accesses run in order
  }
}

struct Ws {
  uint16_t *wglu, *wout, *wgate;
  float *oglu, *oout, *ogate;
  uint16_t *a, *b, *t;
  size_t bytes;
};

Ws carve(char* base, int N) {
  Ws w{};
  size_t off = 0;
  auto take = [&](size_t bytes) { char* p = base ? base + off : nullptr; off += align256(bytes); return p; };
  const size_t ab = (size_t)padded_n(N) * padded_n(N) * kC * 2;      // a / b planes, [c][Pn][Pn]
  const size_t tp = (size_t)plane_stride(N) * kC * 2;                 // t planes, [c][Pp]
  w.wglu = reinterpret_cast<uint16_t*>(take((size_t)kGlu * kC * 2));
  w.wout = reinterpret_cast<uint16_t*>(take((size_t)kC * kC * 2));
  w.wgate = reinterpret_cast<uint16_t*>(take((size_t)kC * kC * 2));
  w.oglu = reinterpret_cast<float*>(take(kGlu * 4));
  w.oout = reinterpret_cast<float*>(take(kC * 4));
  w.ogate = reinterpret_cast<float*>(take(kC * 4));
  w.a = reinterpret_cast<uint16_t*>(take(ab));
  w.b = reinterpret_cast<uint16_t*>(take(ab));
  w.t = reinterpret_cast<uint16_t*>(take(tp));
  w.bytes = off;
  return w;
}

size_t ws_bytes(int N) { return carve(nullptr, N).bytes; }

int launch_grid(const void* kernel, int items) {
  const int waves = std::max(1, std::min(sf_resident_workgroups(kernel, 64 * kTW) * kTW, items));
  return waves;
}

}  // namespace

extern "C" size_t sf_hip_triangle_mult_workspace_bytes(int32_t N, int32_t C) {
  if (N <= 0 || C != kC) return 0;
  return ws_bytes(N);
}

extern "C" int sf_hip_triangle_mult_fwd(const sf_triangle_mult_args* a, void* workspace, size_t workspace_bytes,
                                        void* stream) {
  if (a == nullptr || a->z == nullptr || a->out == nullptr || a->w_glu == nullptr || a->w_out == nullptr ||
      a->w_gate == nullptr || a->cn_w == nullptr || a->ln_w == nullptr) {
    sf_set_error("triangle_mult: z, out, the three weights, ln_w and cn_w must be non-null");
    return 1;
  }
  if (a->C != kC || a->N <= 0 || a->N > 8192) {
    sf_set_error("triangle_mult: need C == %d and 0 < N <= 8192 (N=%d C=%d)", kC, a->N, a->C);
    return 1;
  }
  if (a->z == a->out) {
    sf_set_error("triangle_mult: out may not alias z");
    return 1;
  }
  if (workspace == nullptr || workspace_bytes < ws_bytes(a->N)) {
    sf_set_error("triangle_mult: workspace of %zu bytes needed, %zu given", ws_bytes(a->N), workspace_bytes);
    return 1;
  }
  if (((reinterpret_cast<uintptr_t>(a->z) | reinterpret_cast<uintptr_t>(a->out) |
        reinterpret_cast<uintptr_t>(a->w_glu) | reinterpret_cast<uintptr_t>(a->w_out) |
        reinterpret_cast<uintptr_t>(a->w_gate)) & 15) != 0) {
    sf_set_error("triangle_mult: z, out and the weights must be 16-byte aligned");
    return 1;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int N = a->N, Pn = padded_n(N);
  const int64_t P = (int64_t)N * N, Pp = plane_stride(N);
  const Ws w = carve(static_cast<char*>(workspace), N);

  FoldArgs f{};
  f.w[0] = static_cast<const uint16_t*>(a->w_glu); f.g[0] = a->ln_w; f.b[0] = a->ln_b; f.rows[0] = kGlu;
  f.wf[0] = w.wglu; f.off[0] = w.oglu;
  f.w[1] = static_cast<const uint16_t*>(a->w_out); f.g[1] = a->cn_w; f.b[1] = a->cn_b; f.rows[1] = kC;
  f.wf[1] = w.wout; f.off[1] = w.oout;
  f.w[2] = static_cast<const uint16_t*>(a->w_gate); f.g[2] = a->ln_w; f.b[2] = a->ln_b; f.rows[2] = kC;
  f.wf[2] = w.wgate; f.off[2] = w.ogate;
  hipLaunchKernelGGL(trimul_fold_kernel, dim3((kGlu + 2 * kC + 3) / 4), dim3(256), 0, st, f);   // a wave per row
  int rc = sf_check_launch("trimul_fold_kernel");
  if (rc) return rc;

  {
    ProjArgs pa{};
    pa.N = N; pa.Pn = Pn; pa.incoming = a->incoming ? 1 : 0;
    pa.z = static_cast<const uint16_t*>(a->z); pa.mask = a->mask;
    pa.w = w.wglu; pa.off = w.oglu; pa.a = w.a; pa.b = w.b;
    pa.items = Pn * (Pn / 32);                          // every plane row, padding included
    const int waves = launch_grid(reinterpret_cast<const void*>(trimul_proj_kernel), pa.items);
    pa.items_per_wave = (pa.items + waves - 1) / waves;
    const int groups = (pa.items + pa.items_per_wave * kTW - 1) / (pa.items_per_wave * kTW);
    hipLaunchKernelGGL(trimul_proj_kernel, dim3(groups), dim3(64 * kTW), 0, st, pa);
    if ((rc = sf_check_launch("trimul_proj_kernel"))) return rc;
  }

  // t[c][i][j] = sum_k A[c][i][k] B[c][j][k], rows i, j < N, contraction over the padded Pn
  {
    sf_linear_args g{};
    g.M = N; g.N = N; g.K = Pn;
    g.x = a->incoming ? w.b : w.a; g.x_rs = Pn;
    g.wt = a->incoming ? w.a : w.b;
    g.mul_rows = 1;
    g.y = w.t; g.y_rs = N;
    g.batch = kC; g.x_bs = (int64_t)Pn * Pn; g.w_bs = (int64_t)Pn * Pn; g.y_bs = Pp;
    if ((rc = sf_hip_linear_fwd(&g, st))) return rc;
  }

  const int items = (int)((P + 31) / 32);              // 32-position blocks of the output
  OutArgs oa{};
  oa.P = P; oa.Pp = Pp; oa.t = w.t; oa.z = static_cast<const uint16_t*>(a->z);
  oa.wo = w.wout; oa.oo = w.oout; oa.wg = w.wgate; oa.og = w.ogate;
  oa.add_residual = a->add_residual; oa.out = static_cast<uint16_t*>(a->out); oa.items = items;
  const int waves = launch_grid(reinterpret_cast<const void*>(trimul_out_kernel), items);
  oa.items_per_wave = (items + waves - 1) / waves;
  const int groups = (items + oa.items_per_wave * kTW - 1) / (oa.items_per_wave * kTW);
  hipLaunchKernelGGL(trimul_out_kernel, dim3(groups), dim3(64 * kTW), 0, st, oa);
  return sf_check_launch("trimul_out_kernel");
}
