"""HIP row kernels (LayerNorm / AdaLN, linear epilogues, pair logits, window gather) vs
float32 torch on the same bf16 inputs."""
import pytest
import torch

from oracle.modules import atom_layout_convert
from oracle.primitives import layer_norm as oracle_ln
from sparsefold_amd.backends.hip import ops
from sparsefold_amd import workloads as W
from tests._metrics import BF16_ULP, assert_close_bf16, bf16_round

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("M,C", [(1, 8), (37, 128), (300, 384), (65, 768), (9, 2048)])
def test_layer_norm_affine(M, C):
  g = torch.Generator().manual_seed(M + C)
  x = (torch.randn(M, C, generator=g) * 2 + 0.5).to(torch.bfloat16)
  w, b = 1 + 0.1 * torch.randn(C, generator=g), 0.1 * torch.randn(C, generator=g)
  out = ops.layer_norm(x.to(DEV), w.to(DEV), b.to(DEV))
  ref = oracle_ln(x.float(), w, b)
  assert_close_bf16(out, ref, f"layer_norm {M}x{C}")


def test_layer_norm_adaptive_rows_broadcast():
  g = torch.Generator().manual_seed(3)
  x = torch.randn(3, 50, 64, generator=g).to(torch.bfloat16)
  scale = torch.rand(50, 64, generator=g).to(torch.bfloat16)
  shift = torch.randn(50, 64, generator=g).to(torch.bfloat16)
  out = ops.layer_norm(x.to(DEV), scale=scale.to(DEV), shift=shift.to(DEV))
  ref = oracle_ln(x.float(), None, None) * scale.float() + shift.float()
  assert_close_bf16(out, ref, "adaln")


# Shapes cover both GEMM kernels (K % 64 != 0 and == 0), each tile size of the K % 64 == 0
# kernel (64x64, 64x128 at >= 512 tiles, 128x128 at >= 512 tiles), odd K-step counts, ragged
# M / N edges (N % 4 != 0 exercises the partial 4-column epilogue group) and the diffusion
# projection's 5120 x 3072 x 768.
@pytest.mark.parametrize("M,N,K", [(1, 8, 8), (100, 96, 128), (257, 516, 128), (1030, 384, 384), (64, 3072, 768),
                                   (1, 8, 64), (130, 70, 64), (4100, 1030, 192), (32773, 256, 128), (77, 3, 320),
                                   (4100, 3610, 192), (5120, 3072, 768), (14700, 1030, 64)])
def test_linear_plain(M, N, K):
  g = torch.Generator().manual_seed(M * 7 + N)
  x = torch.randn(M, K, generator=g).to(torch.bfloat16)
  w = (torch.randn(N, K, generator=g) / K ** 0.5).to(torch.bfloat16)
  out = ops.linear(x.to(DEV), w.to(DEV))
  ref = x.float() @ w.float().t()
  assert_close_bf16(out, ref, f"linear {M}x{N}x{K}")


@pytest.mark.parametrize("K", [64, 72])
def test_linear_epilogue_bias_sigmoid_mul_residual_and_transposed_columns(K):
  g = torch.Generator().manual_seed(9)
  M, N = 300, 72
  x = torch.randn(M, K, generator=g).to(torch.bfloat16)
  w = (torch.randn(N, K, generator=g) / 8).to(torch.bfloat16)
  bias = torch.randn(N, generator=g)
  mul = torch.randn(100, N, generator=g).to(torch.bfloat16)
  res = torch.randn(M, N, generator=g).to(torch.bfloat16)
  yt = torch.empty(8, M, dtype=torch.bfloat16, device=DEV)
  out = ops.linear(x.to(DEV), w.to(DEV), bias.to(DEV), post_sigmoid=True, mul=mul.to(DEV), residual=res.to(DEV),
                   yt=yt, tcol0=64)
  pre = torch.sigmoid(x.float() @ w.float().t() + bias)
  ref = pre * mul.float().repeat(3, 1) + res.float()
  assert_close_bf16(out, ref, "linear epilogue")
  assert_close_bf16(yt, ref[:, 64:72].t(), "linear transposed columns")
  y2 = ops.linear(x.to(DEV), w.to(DEV), ycols=64)
  assert y2.shape == (M, 64)
  assert_close_bf16(y2, x.float() @ w.float()[:64].t(), "linear ycols")


def test_linear_large_epilogues():
  """A large ragged product (4100 x 3608, 128x128 tiles) under every epilogue: bias, sigmoid,
  row-broadcast multiplier, residual, transposed columns and ycols, and the gated pairs."""
  g = torch.Generator().manual_seed(11)
  M, N, K = 4100, 3608, 128
  x = torch.randn(M, K, generator=g).to(torch.bfloat16)
  w = (torch.randn(N, K, generator=g) / 8).to(torch.bfloat16)
  bias = torch.randn(N, generator=g)
  mul = torch.randn(41, N, generator=g).to(torch.bfloat16)
  res = torch.randn(M, N, generator=g).to(torch.bfloat16)
  yt = torch.empty(16, M, dtype=torch.bfloat16, device=DEV)
  out = ops.linear(x.to(DEV), w.to(DEV), bias.to(DEV), post_sigmoid=True, mul=mul.to(DEV), residual=res.to(DEV),
                   yt=yt, tcol0=3000)
  pre = torch.sigmoid(x.float() @ w.float().t() + bias)
  ref = pre * mul.float().repeat(M // 41 + 1, 1)[:M] + res.float()
  assert_close_bf16(out, ref, "linear large epilogue")
  assert_close_bf16(yt, ref[:, 3000:3016].t(), "linear large transposed columns")
  y2 = ops.linear(x.to(DEV), w.to(DEV), ycols=3500)
  assert y2.shape == (M, 3500)
  assert_close_bf16(y2, x.float() @ w.float()[:3500].t(), "linear large ycols")
  # gated pairs (C ABI): output column j = swish(col 2j) * col 2j + 1
  import ctypes
  from sparsefold_amd import _lib
  w = (w.float() / 4).to(torch.bfloat16)           # products of O(1) gates and values
  bias = bias / 4
  xd, wd, bd = x.to(DEV), w.to(DEV), bias.to(DEV)
  yg = torch.empty(M, N // 2, dtype=torch.bfloat16, device=DEV)
  a = _lib.LinearArgs()
  a.M, a.N, a.K = M, N, K
  a.x, a.x_rs, a.wt, a.bias = xd.data_ptr(), K, wd.data_ptr(), bd.data_ptr()
  a.y, a.y_rs, a.mul_rows, a.glu = yg.data_ptr(), N // 2, 1, 1
  _lib.check(_lib.load().sf_hip_linear_fwd(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
             "sf_hip_linear_fwd")
  h = x.float() @ w.float().t() + bias
  assert_close_bf16(yg, torch.nn.functional.silu(h[:, 0::2]) * h[:, 1::2], "linear large glu")


# C = 128 runs the MFMA kernel (P = 1320: a ragged last 32-position step, 16-byte stores; P = 1517:
# P % 8 != 0, 2-byte stores); other C the per-position kernel.  H = 100, 130, 200 with 16-byte
# stores: tiles whose last planes lie past H (their lanes store the last valid plane again), and
# the one-tile-per-workgroup layout where a second tile would hold no plane (H = 130).
@pytest.mark.parametrize("H,C,with_b,shape", [(4, 128, True, (33, 40)), (16, 128, True, (33, 40)),
                                              (16, 128, True, (37, 41)), (12, 16, False, (33, 40)),
                                              (64, 128, False, (33, 40)), (40, 128, True, (37, 41)),
                                              (100, 128, True, (37, 41)), (384, 128, False, (64, 64)),
                                              (100, 128, False, (33, 40)), (130, 128, True, (33, 40)),
                                              (200, 128, False, (33, 40))])
def test_pair_logits(H, C, with_b, shape):
  g = torch.Generator().manual_seed(H * C)
  z = torch.randn(*shape, C, generator=g).to(torch.bfloat16)
  lw, lb = 1 + 0.1 * torch.randn(C, generator=g), 0.1 * torch.randn(C, generator=g)
  w = (torch.randn(H, C, generator=g) / C ** 0.5).to(torch.bfloat16)
  out = ops.pair_logits(z.to(DEV), lw.to(DEV), lb.to(DEV) if with_b else None, w.to(DEV))
  ref = torch.einsum("abc,hc->hab", oracle_ln(z.float(), lw, lb if with_b else None), w.float()).reshape(H, -1)
  assert_close_bf16(out, ref, f"pair_logits H={H} C={C}", rtol=BF16_ULP)   # bf16 logits planes of O(1-5)


@pytest.mark.parametrize("C,U,QK,blocks,H", [(16, 8, 4096, 3, 4), (128, 6, 35, 3, 4), (128, 3, 64, 12, 8)])
def test_pair_logits_segmented_layout_is_a_permutation(C, U, QK, blocks, H):
  """The segmented store writes exactly the plane-major values, permuted
  [blocks, H, U, QK] -> [blocks, U, H, QK] (same arithmetic, different addresses)."""
  g = torch.Generator().manual_seed(C + QK)
  z = torch.randn(U * QK, C, generator=g).to(torch.bfloat16).to(DEV)
  lw = (1 + 0.1 * torch.randn(C, generator=g)).to(DEV)
  w = (torch.randn(blocks * H, C, generator=g) / C ** 0.5).to(torch.bfloat16).to(DEV)
  flat = ops.pair_logits(z, lw, None, w)
  seg = ops.pair_logits(z, lw, None, w, seg=QK, group=H)
  assert seg.shape == (blocks, U, H, QK)
  assert torch.equal(seg, flat.view(blocks, H, U, QK).permute(0, 2, 1, 3))


def test_window_gather_exact():
  lay = W.window_layout(256, pad=20)
  g = torch.Generator().manual_seed(4)
  act = torch.randn(3, 8, 32, 16, generator=g).to(torch.bfloat16)
  keys = ops.window_gather(act.reshape(3, 256, 16).to(DEV), lay.gather_idxs.to(DEV), lay.gather_mask.to(DEV))
  ref = atom_layout_convert(lay.gather_idxs, lay.gather_mask, (8, 32), act, layout_axes=(-3, -2))
  assert torch.equal(keys.view(3, 8, 128, 16).cpu(), ref)
