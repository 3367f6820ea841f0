// Triangle attention module (starting / ending node) on gfx950.
//
// Replaces GridSelfAttention.forward (src/sparsefold/model/trunk/blocks.py:293-366 with the
// per-chunk _attention of :270-291).  Pipeline, all on one stream:
//   1. layer_norm_kernel    x = LN(z)                                  (blocks.py:317)
//   2. linear_kernel        [q|k|v|g] = x W^T, bias planes [H, N*N]    (blocks.py:276-278,
//                           :286, :320-329; bias kept in the untransposed orientation)
//   3. attention_fwd_kernel rows r of x (x^T for the ending node, read through strides --
//                           nothing is transposed in memory), mask_k = seq[r] & seq[k],
//                           shared bias (row stride 0), sigmoid gate fused
//   4. linear_kernel        out = z + o W_o                             (blocks.py:291, :366)
// The attention output is written at the pair position it belongs to, so the ending node
// needs no transpose back either.
#include <cmath>

#include "sf_common.h"

namespace {
size_t round_up(size_t x) { return (x + 255) & ~(size_t)255; }

struct TriWs {
  uint16_t* xhat;   // [P, C]
  uint16_t* y;      // [P, 4HD]  q | k | v | g
  uint16_t* bias;   // [H, P]
  uint16_t* o;      // [P, HD]
  size_t bytes;
};

TriWs carve(void* base, int32_t N, int32_t C, int32_t H, int32_t D) {
  const size_t P = (size_t)N * N, HD = (size_t)H * D;
  TriWs w{};
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
  return carve(nullptr, N, C, H, D).bytes;
}

extern "C" int sf_hip_triangle_attn_fwd(const sf_triangle_args* a, void* workspace, size_t workspace_bytes,
                                        void* stream) {
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
