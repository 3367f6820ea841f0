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


def _ln_gamma(x, w):
  """LayerNorm with a scale and no offset (the pair_input_layer_norm of both packs)."""
  return layer_norm(x, w, None)


def transformer_pair_logits(pair_cond, p):
  """transformer.py:430-438 written per element: pair_cond ``[N0, N1, P]`` float64 ->
  ``[n_super, S, H, N0, N1]``.  Plane (sb, s, h) at (b, n) is the dot product of the normalised
  pair_cond[b, n] with column (s, h) of super-block sb's projection ``[P, S, H]``."""
  pc = np.asarray(pair_cond, np.float64)
  N0, N1, P = pc.shape
  gamma = np.asarray(p["pair_input_layer_norm.weight"], np.float64)
  ws = []
  while f"pair_logits_projection.{len(ws)}.weight" in p:
    ws.append(np.asarray(p[f"pair_logits_projection.{len(ws)}.weight"], np.float64))
  S, H = ws[0].shape[1:]
  out = np.zeros((len(ws), S, H, N0, N1))
  for b in range(N0):
    for n in range(N1):
      x = _ln_gamma(pc[b, n], gamma)
      for sb, w in enumerate(ws):
        for s in range(S):
          for h in range(H):
            out[sb, s, h, b, n] = sum(x[c] * w[c, s, h] for c in range(P))
  return out


def cross_att_pair_logits(pair_cond, p):
  """transformer.py:655-662 written per element: pair_cond ``[U, Q, K, P]`` float64 ->
  ``[blocks, U, H, Q, K]``.  Plane (blk, h) of window u at (q, k) is the dot product of the
  normalised pair_cond[u, q, k] with column (blk, h) of the projection ``[P, blocks, H]``."""
  pc = np.asarray(pair_cond, np.float64)
  U, Q, K, P = pc.shape
  gamma = np.asarray(p["pair_input_layer_norm.weight"], np.float64)
  w = np.asarray(p["pair_logits_projection.weight"], np.float64)
  nb, H = w.shape[1:]
  out = np.zeros((nb, U, H, Q, K))
  for u in range(U):
    for q in range(Q):
      for k in range(K):
        x = _ln_gamma(pc[u, q, k], gamma)
        for blk in range(nb):
          for h in range(H):
            out[blk, u, h, q, k] = sum(x[c] * w[c, blk, h] for c in range(P))
  return out


def _adaln_row(x, c, p, prefix):
  """AdaLN of one row (transformer.py:80-96): LN(x) scaled by sigmoid(LN_g(c) Ws + bs), shifted
  by LN_g(c) Wb.  Without a condition: LN(x) with the side's own scale and offset."""
  if c is None:
    return layer_norm(x, p[prefix + "layer_norm.weight"], p.get(prefix + "layer_norm.bias"))
  cn = layer_norm(c, p[prefix + "single_cond_layer_norm.weight"], p.get(prefix + "single_cond_layer_norm.bias"))
  ws = np.asarray(p[prefix + "single_cond_scale.weight"], np.float64)
  bs = np.asarray(p[prefix + "single_cond_scale.bias"], np.float64)
  wb = np.asarray(p[prefix + "single_cond_bias.weight"], np.float64)
  C = ws.shape[1]
  xn = layer_norm(x)
  return np.array([sigmoid(sum(cn[m] * ws[m, n] for m in range(len(cn))) + bs[n]) * xn[n]
                   + sum(cn[m] * wb[m, n] for m in range(len(cn))) for n in range(C)])


def cross_attention(x_q, x_k, mask_q, mask_k, p, pair_logits=None, cond_q=None, cond_k=None):
  """transformer.py:549-585 (CrossAttention.forward) written per window, query, key and head in
  float64: x_q ``[U, Q, C]``, x_k ``[U, K, C]``, masks ``[U, Q]`` / ``[U, K]``, pair_logits
  ``[U, H, Q, K]``, conditions ``[U, Q, C]`` / ``[U, K, C]``.  The query side is normalised with
  the ``q_layernorm.`` parameters and its condition, the key side with ``k_layernorm.`` and
  its own; the gate comes from the normalised queries, the AdaLN-zero multiplier from the
  query condition.  Returns (x_q + update, update)."""
  xq = np.asarray(x_q, np.float64)
  xk = np.asarray(x_k, np.float64)
  U, Q, C = xq.shape
  K = xk.shape[1]
  wq = np.asarray(p["q_projection.weight"], np.float64)        # [C, H, D]
  bq = np.asarray(p["q_projection.bias"], np.float64)          # [H, D]
  wk = np.asarray(p["k_projection.weight"], np.float64)
  wv = np.asarray(p["v_projection.weight"], np.float64)
  wg = np.asarray(p["gating_query.weight"], np.float64)        # [C, H*D]
  wt = np.asarray(p["zero_init.transition2.weight"], np.float64)   # [H*D, C]
  H, D = wq.shape[1:]
  upd = np.zeros_like(xq)
  for u in range(U):
    hq = [_adaln_row(xq[u, i], None if cond_q is None else np.asarray(cond_q[u, i], np.float64), p, "q_layernorm.")
          for i in range(Q)]
    hk = [_adaln_row(xk[u, j], None if cond_k is None else np.asarray(cond_k[u, j], np.float64), p, "k_layernorm.")
          for j in range(K)]
    for i in range(Q):
      o = np.zeros(H * D)
      for h in range(H):
        q = np.array([sum(hq[i][c] * wq[c, h, d] for c in range(C)) + bq[h, d] for d in range(D)])
        ks = [np.array([sum(hk[j][c] * wk[c, h, d] for c in range(C)) for d in range(D)]) for j in range(K)]
        vs = [np.array([sum(hk[j][c] * wv[c, h, d] for c in range(C)) for d in range(D)]) for j in range(K)]
        valid = [bool(mask_q[u, i]) and bool(mask_k[u, j]) for j in range(K)]
        logits = [sum(q[d] * ks[j][d] for d in range(D)) / np.sqrt(D)
                  + (0.0 if pair_logits is None else float(pair_logits[u, h, i, j])) for j in range(K)]
        if any(valid):
          m = max(l for l, ok in zip(logits, valid) if ok)
          e = [np.exp(l - m) if ok else 0.0 for l, ok in zip(logits, valid)]
        else:
          e = [1.0] * K                                        # every logit is the same -max
        tot = sum(e)
        for d in range(D):
          o[h * D + d] = sum(e[j] * vs[j][d] for j in range(K)) / tot
      g = np.array([sigmoid(sum(hq[i][c] * wg[c, n] for c in range(C))) for n in range(H * D)])
      y = np.array([sum(o[n] * g[n] * wt[n, c] for n in range(H * D)) for c in range(C)])
      if cond_q is not None:
        cq = np.asarray(cond_q[u, i], np.float64)
        wz = np.asarray(p["zero_init.adaptive_zero_cond.weight"], np.float64)
        bz = np.asarray(p["zero_init.adaptive_zero_cond.bias"], np.float64)
        y = y * np.array([sigmoid(sum(cq[m] * wz[m, c] for m in range(len(cq))) + bz[c]) for c in range(C)])
      upd[u, i] = y
  return xq + upd, upd


def _swish(v):
  return v * sigmoid(v)


def transition_block(act, p):
  """blocks.py:84-96 per row and channel in float64: act ``[R, C]``.  Returns (act + upd, upd)."""
  act = np.asarray(act, np.float64)
  R, C = act.shape
  w1 = np.asarray(p["transition1.weight"], np.float64)        # [C, 2I]: a = cols [0, I), b = [I, 2I)
  w2 = np.asarray(p["transition2.weight"], np.float64)        # [I, C]
  I = w2.shape[0]
  upd = np.zeros_like(act)
  for r in range(R):
    x = layer_norm(act[r], p["input_layer_norm.weight"], p.get("input_layer_norm.bias"))
    c = [_swish(sum(x[m] * w1[m, i] for m in range(C))) * sum(x[m] * w1[m, I + i] for m in range(C))
         for i in range(I)]
    upd[r] = [sum(c[i] * w2[i, n] for i in range(I)) for n in range(C)]
  return act + upd, upd


def diffusion_transition_block(x, cond, p):
  """transformer.py:209-231 per row and channel in float64: x ``[R, C]``, cond ``[R, Cs]`` or
  None.  Returns (x + upd, upd)."""
  x = np.asarray(x, np.float64)
  R, C = x.shape
  w1 = np.asarray(p["transition.weight"], np.float64)
  w2 = np.asarray(p["zero_init.transition2.weight"], np.float64)
  I = w2.shape[0]
  upd = np.zeros_like(x)
  for r in range(R):
    c_row = None if cond is None else np.asarray(cond[r], np.float64)
    h = _adaln_row(x[r], c_row, p, "layer_norm.")
    c = [_swish(sum(h[m] * w1[m, i] for m in range(C))) * sum(h[m] * w1[m, I + i] for m in range(C))
         for i in range(I)]
    y = np.array([sum(c[i] * w2[i, n] for i in range(I)) for n in range(C)])
    if c_row is not None:
        wz = np.asarray(p["zero_init.adaptive_zero_cond.weight"], np.float64)
        bz = np.asarray(p["zero_init.adaptive_zero_cond.bias"], np.float64)
        y = y * np.array([sigmoid(sum(c_row[m] * wz[m, n] for m in range(len(c_row))) + bz[n]) for n in range(C)])
    upd[r] = y
  return x + upd, upd
