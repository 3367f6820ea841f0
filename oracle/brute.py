"""Float64 numpy loop implementations that pin the torch restatement.

TEST INFRASTRUCTURE: imported only by tests.

These share no code with torch's SDPA: logits, masking and softmax are written
out per (batch, head, query).  The masking rule is the one the reference's
arithmetic produces (sdpa.py:62-80, masked logits set to ``-finfo.max``): keys
masked for a query get weight 0, and a query with *no* valid key weighs every
key equally (all its logits are the same ``-max``).
"""
from __future__ import annotations

import numpy as np


def attention(q, k, v, scale=None, mask_q=None, mask_k=None, bias=None):
  """q ``[B,Q,H,D]``, k ``[B,K,H,D]``, v ``[B,K,H,Dv]``, mask_q ``[B,Q]``,
  mask_k ``[B,K]``, bias ``[B,H,Q,K]`` (already broadcast).  float64."""
  q = np.asarray(q, np.float64)
  k = np.asarray(k, np.float64)
  v = np.asarray(v, np.float64)
  B, Q, H, D = q.shape
  K = k.shape[1]
  Dv = v.shape[-1]
  s = 1.0 / np.sqrt(D) if scale is None else scale
  out = np.zeros((B, Q, H, Dv))
  for b in range(B):
    for h in range(H):
      for i in range(Q):
        logits = np.array([s * float(np.dot(q[b, i, h], k[b, j, h])) for j in range(K)])
        if bias is not None:
          logits = logits + np.asarray(bias[b, h, i], np.float64)
        valid = np.ones(K, bool)
        if mask_k is not None:
          valid &= np.asarray(mask_k[b], bool)
        if mask_q is not None and not bool(mask_q[b, i]):
          valid[:] = False
        if not valid.any():
          w = np.full(K, 1.0 / K)
        else:
          m = logits[valid].max()
          e = np.where(valid, np.exp(logits - m), 0.0)
          w = e / e.sum()
        out[b, i, h] = w @ v[b, :, h]
  return out


def layer_norm(x, w=None, b=None, eps=1e-5):
  x = np.asarray(x, np.float64)
  mu = x.mean(-1, keepdims=True)
  var = ((x - mu) ** 2).mean(-1, keepdims=True)
  y = (x - mu) / np.sqrt(var + eps)
  if w is not None:
    y = y * np.asarray(w, np.float64)
  if b is not None:
    y = y + np.asarray(b, np.float64)
  return y


def sigmoid(x):
  return 1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))


def grid_self_attention(act, seq_mask, p, transpose):
  """Triangle attention written per row: act ``[N,N,C]`` float64 result."""
  z = np.asarray(act, np.float64)
  N = z.shape[0]
  wq = np.asarray(p["q_projection.weight"], np.float64)        # [H,D,C]
  wk = np.asarray(p["k_projection.weight"], np.float64)        # [H,D,C]
  wv = np.asarray(p["v_projection.weight"], np.float64)        # [C,H,D]
  wg = np.asarray(p["gating_query.weight"], np.float64)        # [H*D,C]
  wo = np.asarray(p["output_projection.weight"], np.float64)   # [H*D,C]
  wb = np.asarray(p["pair_bias_projection.weight"], np.float64)  # [C,H]
  H, D, _ = wq.shape
  lb = p.get("act_norm.bias")
  x = layer_norm(z, p["act_norm.weight"], lb)
  bias = np.einsum("qkc,ch->hqk", x, wb)                       # untransposed orientation
  xt = x.transpose(1, 0, 2) if transpose else x
  seq = np.asarray(seq_mask, bool)
  upd = np.zeros_like(z)
  for r in range(N):
    xr = xt[r]                                                  # [N, C]
    q = np.einsum("nc,hdc->nhd", xr, wq)
    k = np.einsum("nc,hdc->nhd", xr, wk)
    v = np.einsum("nc,chd->nhd", xr, wv)
    mk = seq[r] & seq
    o = attention(q[None], k[None], v[None], mask_k=mk[None], bias=bias[None])[0]
    g = sigmoid(xr @ wg.T)
    u = (o.reshape(N, H * D) * g) @ wo
    if transpose:
      upd[:, r] = u
    else:
      upd[r] = u
  return z + upd, upd


def triangle_multiplication(act, mask, p, incoming):
  """blocks.py:486-566 written out per position and channel: act ``[N, N, C]`` float64, mask
  ``[N]`` bool, p the module's float weights (Linear weights ``[in, out]``).  Returns
  (act + update, update)."""
  act = np.asarray(act, np.float64)
  N, _, C = act.shape
  x = np.zeros_like(act)
  for i in range(N):
    for k in range(N):
      x[i, k] = layer_norm(act[i, k], p["left_norm_input.weight"], p.get("left_norm_input.bias"))
  wg = np.asarray(p["gate_projection.weight"], np.float64)
  wp = np.asarray(p["projection.weight"], np.float64)
  # projected channel ch = 2c + side: side 0 feeds a, side 1 feeds b ("(c i2) ..." split)
  a = np.zeros((C, N, N))
  b = np.zeros((C, N, N))
  for i in range(N):
    for k in range(N):
      if not (mask[i] and mask[k]):
        continue
      for ch in range(2 * C):
        g = sum(x[i, k, m] * wg[m, ch] for m in range(C))
        v = sum(x[i, k, m] * wp[m, ch] for m in range(C))
        (a if ch % 2 == 0 else b)[ch // 2, i, k] = sigmoid(g) * v
  t = np.zeros((N, N, C))
  for c in range(C):
    for i in range(N):
      for j in range(N):
        if incoming:
          t[i, j, c] = sum(a[c, k, j] * b[c, k, i] for k in range(N))
        else:
          t[i, j, c] = sum(a[c, i, k] * b[c, j, k] for k in range(N))
  wo = np.asarray(p["output_projection.weight"], np.float64)
  wgl = np.asarray(p["gating_linear.weight"], np.float64)
  upd = np.zeros_like(act)
  for i in range(N):
    for j in range(N):
      tn = layer_norm(t[i, j], p["center_norm.weight"], p.get("center_norm.bias"))
      gate = np.array([sigmoid(sum(x[i, j, m] * wgl[m, n] for m in range(C))) for n in range(C)])
      upd[i, j] = np.array([sum(tn[m] * wo[m, n] for m in range(C)) for n in range(C)]) * gate
  return act + upd, upd
