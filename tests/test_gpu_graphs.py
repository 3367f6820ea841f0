"""HIP-graph replay of repeated module calls: every replay must equal the eager call exactly
(same kernels), with eager work and synchronisations between replays; new values at a captured
address are seen; new addresses run eagerly; re-packing the weights drops the graphs."""
import pytest
import torch

from sparsefold_amd import backends
from sparsefold_amd import workloads as W
from sparsefold_amd.backends.hip import graphs
from sparsefold_amd.runtime import config

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def hip_backend():
  config.configure_runtime(backend="hip", sdpa_implementation="hip", device="cuda")
  backends.init()
  yield
  config.configure_runtime(backend="torch")
  backends.init()
  config.reset()


def _set_graphs(on: bool):
  config.configure_runtime(backend="hip", sdpa_implementation="hip", device="cuda", hip_graphs=on)


def _cases():
  def tri():
    mod, z, seq = W.make_triangle(96, padded=True, seed=21)
    return mod, (z.to(DEV), seq.to(DEV)), {}
  def single():
    mod, z, s, seq = W.make_single(96, seed=22, padded=True)
    return mod, (z.to(DEV), s.to(DEV), seq.to(DEV)), {}
  def diffusion():
    mod, act, cond, bias, mask = W.make_diffusion(128, S=2, seed=23, padded=True)
    return mod, (act.to(DEV), mask.to(DEV)), {"pair_logits": bias.to(DEV), "single_cond": cond.to(DEV)}
  def window():
    mod, act, lay, qc, kc, bias = W.make_window(256, S=2, seed=24, pad=20)
    args = tuple(x.to(DEV) for x in (act, lay.queries_mask, lay.gather_idxs, lay.gather_mask, lay.keys_mask, qc, kc, bias))
    return mod, args, {"_method": "forward_indexed"}
  return {"triangle": tri, "single": single, "diffusion": diffusion, "window": window}


@pytest.mark.parametrize("name", ["triangle", "single", "diffusion", "window"])
def test_graph_replay_matches_eager(name):
  mod, args, kwargs = _cases()[name]()
  method = kwargs.pop("_method", "forward")
  mod = mod.to(DEV)
  backends.prepare(mod)
  call = lambda: getattr(mod, method)(*args, **kwargs)
  _set_graphs(False)
  ref = call().clone()
  torch.cuda.synchronize()
  _set_graphs(True)
  scratch = torch.randn(1 << 20, device=DEV)
  outs = []
  for i in range(5):                                   # eager, capture + replay, then replays
    outs.append(call())
    scratch.mul_(1.0001).add_(float(i))                # the program's own eager work between replays
    torch.cuda.synchronize()
  cache = mod.__dict__.get("_hip_graph_cache", {})
  assert any(v is not graphs._SEEN for v in cache.values()), "no graph was captured"
  for i, out in enumerate(outs):
    assert torch.equal(out, ref), f"{name}: call {i} differs from the eager result"
  # the returned tensor is a copy: a later replay does not change an earlier result
  first = outs[2]
  call()
  torch.cuda.synchronize()
  assert torch.equal(first, ref)
  # new values at the captured address are read by the replay
  x0 = args[0]
  x0.mul_(0.5)
  _set_graphs(False)
  ref2 = call().clone()
  _set_graphs(True)
  assert torch.equal(call(), ref2)
  # new tensors (new addresses): eager first, then equal again
  new_args = tuple(a.clone() if isinstance(a, torch.Tensor) else a for a in args)
  out_new = getattr(mod, method)(*new_args, **kwargs)
  assert torch.equal(out_new, ref2)
  # re-packing the weights drops the graphs
  backends.prepare(mod)
  assert "_hip_graph_cache" not in mod.__dict__
  assert torch.equal(call(), ref2)
  _set_graphs(False)
