"""Plugin boundary on the CPU: runtime selection keys, backend lifecycle, factory
replacement, preparation guards (mirrors tests/test_runtime_reference.py and
tests/test_native_preparation.py of the reference)."""
import pytest
import torch

from sparsefold_amd import backends
from sparsefold_amd import modules as M
from sparsefold_amd.runtime import config


def test_configure_runtime_accepts_hip_selection_keys(reset_runtime):
  config.configure_runtime(backend="hip", sdpa_implementation="hip", device="cuda")
  assert config.acclib_implementation == "hip" and config.sdpa_implementation == "hip"
  config.configure_runtime(backend="none")
  assert config.acclib_implementation == "torch"
  with pytest.raises(ValueError, match="SDPA"):
    config.configure_runtime(sdpa_implementation="triton")
  with pytest.raises(TypeError, match="Unknown runtime settings"):
    config.configure_runtime(not_a_setting=1)
  with pytest.raises(ValueError, match="either backend"):
    config.configure_runtime(backend="hip", acclib_implementation="hip")
  opts = config.get_runtime_options()
  opts["native_ops"].append("x")
  assert "x" not in config.native_ops


def test_environment_selection(monkeypatch, reset_runtime):
  monkeypatch.setenv("SPARSEFOLD_ACCLIB_IMPLEMENTATION", "hip")
  monkeypatch.setenv("SPARSEFOLD_SDPA_IMPLEMENTATION", "hip")
  config.reset()
  assert config.acclib_implementation == "hip" and config.sdpa_implementation == "hip"


def test_hip_backend_requires_gpu_device(reset_runtime):
  config.configure_runtime(backend="hip", device="cpu")
  with pytest.raises(RuntimeError, match="GPU only"):
    backends.init()


def test_unknown_native_op_rejected(reset_runtime):
  config.configure_runtime(backend="hip", device="cuda", native_ops=["not_an_op"])
  with pytest.raises(ValueError, match="Unknown native operators"):
    backends.init()


def test_apply_replaces_and_restores_factories(reset_runtime):
  original = M.GridSelfAttention
  config.configure_runtime(backend="hip", device="cuda", native_ops=["grid_self_attn"])
  backends.init()
  assert M.GridSelfAttention is not original and issubclass(M.GridSelfAttention, original)
  assert M.SelfAttention.__name__ == "SelfAttention"          # not selected
  assert M.TransformerPairLogits.__name__ == "TransformerPairLogits"
  config.configure_runtime(backend="torch")
  backends.init()
  config.configure_runtime(backend="hip", device="cuda", native_ops=["diffusion_self_attention"])
  backends.init()
  assert M.SelfAttention.__name__ == "SelfAttentionHip"
  assert M.TransformerPairLogits.__name__ == "TransformerPairLogitsHip"
  assert M.CrossAttTransformerPairLogits.__name__ == "CrossAttTransformerPairLogits"
  config.configure_runtime(backend="torch")
  backends.init()
  assert M.GridSelfAttention is original
  assert backends.prepare(torch.nn.Linear(2, 2)) == {"packed": 0, "fallback": 0, "opaque": 0}


def test_vecops_is_declared_but_unavailable(reset_runtime):
  assert "vecops" in backends.available_libraries() and "hip" in backends.available_libraries()
  config.configure_runtime(backend="vecops", device="cpu")
  with pytest.raises(RuntimeError, match="vecops"):
    backends.init()


def test_unreplaced_modules_have_no_torch_path(reset_runtime):
  mod = M.GridSelfAttention(M.GridSelfAttention.Config(), M.GlobalConfig(), False, num_channels=32, name="x")
  with pytest.raises(RuntimeError, match="no Torch compute path"):
    mod(torch.zeros(4, 4, 32), torch.ones(4, dtype=torch.bool))


def test_reference_parameter_layouts():
  g = M.GridSelfAttention(M.GridSelfAttention.Config(num_head=4), M.GlobalConfig(), False, num_channels=128, name="t")
  shapes = {k: tuple(v.shape) for k, v in g.state_dict().items()}
  assert shapes == {
      "q_projection.weight": (4, 32, 128), "k_projection.weight": (4, 32, 128), "v_projection.weight": (128, 4, 32),
      "gating_query.weight": (128, 128), "output_projection.weight": (128, 128), "act_norm.weight": (128,),
      "pair_bias_projection.weight": (128, 4)}
  s = M.SelfAttention(M.SelfAttention.Config(num_head=16), M.GlobalConfig(), num_channels=768, single_cond_size=384)
  shapes = {k: tuple(v.shape) for k, v in s.state_dict().items()}
  assert shapes["layer_norm.single_cond_scale.weight"] == (384, 768)
  assert shapes["q_projection.weight"] == (768, 16, 48) and shapes["q_projection.bias"] == (16, 48)
  assert shapes["zero_init.adaptive_zero_cond.weight"] == (384, 768)
  assert "layer_norm.layer_norm.weight" not in shapes
  c = M.CrossAttention(M.CrossAttention.Config(), M.GlobalConfig(), num_channels=128)
  assert tuple(c.state_dict()["k_layernorm.single_cond_scale.weight"].shape) == (128, 128)
  u = M.SingleActUpdate(M.GlobalConfig(), 128, 384, M.SelfAttention.Config(num_head=16))
  assert u.single_attention.key_dim == 24
  assert tuple(u.state_dict()["single_pair_logits_projection.weight"].shape) == (128, 16)
  t = M.TransformerPairLogits(num_blocks=24, super_block_size=4, num_head=16, pair_cond_size=128)
  shapes = {k: tuple(v.shape) for k, v in t.state_dict().items()}
  assert shapes == {**{f"pair_logits_projection.{i}.weight": (128, 4, 16) for i in range(6)},
                    "pair_input_layer_norm.weight": (128,)}
  x = M.CrossAttTransformerPairLogits(num_blocks=3, num_head=4, pair_cond_size=16)
  shapes = {k: tuple(v.shape) for k, v in x.state_dict().items()}
  assert shapes == {"pair_logits_projection.weight": (16, 3, 4), "pair_input_layer_norm.weight": (16,)}


def test_prepare_rejects_host_parameters_and_forward_requires_prepare(reset_runtime):
  config.configure_runtime(backend="hip", device="cuda")
  backends.init()
  mod = M.GridSelfAttention(M.GridSelfAttention.Config(), M.GlobalConfig(), False, num_channels=32, name="x")
  with pytest.raises(RuntimeError, match="not prepared"):
    mod(torch.zeros(4, 4, 32), torch.ones(4, dtype=torch.bool))
  with pytest.raises(RuntimeError, match="on the GPU"):
    backends.prepare(mod)


class _ValueCache:
  """Behaviour of the reference ValueCache.get (runtime/cache.py:21-39): keyed by the
  positional arguments' identities and the entry name; with caching off it calls the factory."""

  def __init__(self, enabled: bool = True):
    self.enabled, self.store = enabled, {}

  def get(self, *args, name=None, factory=None):
    if not self.enabled:
      return factory()
    key = (tuple(id(a) for a in args), name)
    if self.store.get(key) is None and factory is not None:
      self.store[key] = factory()
    return self.store.get(key)

  def reset(self):
    self.store.clear()


class _TransformerForward(torch.nn.Module):
  """The cache use of Transformer.forward (transformer.py:430-447) plus one unrelated entry."""

  def __init__(self, enabled: bool = True):
    super().__init__()
    self._cache = _ValueCache(enabled)

  def forward(self, act, mask, single_cond, pair_cond=None):
    pack = None if pair_cond is None else self._cache.get(name="pair_logits", factory=lambda: "reference pack")
    return pack, self._cache.get(name="other", factory=lambda: "other")


@pytest.mark.parametrize("enabled", [True, False])
def test_transformer_pack_replaces_only_the_pair_logit_factory(enabled):
  from sparsefold_amd.backends.hip.modules import TransformerHipMixin
  calls = []

  class Hip(TransformerHipMixin, _TransformerForward):
    def pair_logits_pack(self, pair_cond):
      calls.append(pair_cond)
      return "hip pack"

  mod = Hip(enabled)
  cache = mod._cache
  pc = torch.zeros(2, 2, 4)
  assert mod(None, None, None, pc) == ("hip pack", "other")
  assert mod(None, None, None, pc) == ("hip pack", "other")
  assert len(calls) == (1 if enabled else 2)              # cached once per example when enabled
  assert mod._cache is cache                              # the reference cache object is restored
  assert mod(None, None, None, None) == (None, "other")
  cache.reset()
  mod(None, None, None, pc)
  assert len(calls) == (2 if enabled else 3)


def test_graph_replay_flag_and_signature(monkeypatch, reset_runtime):
  from sparsefold_amd.backends.hip import graphs
  monkeypatch.setenv("SPARSEFOLD_HIP_GRAPHS", "1")
  config.reset()
  assert config.hip_graphs is True
  monkeypatch.delenv("SPARSEFOLD_HIP_GRAPHS")
  config.reset()
  assert config.hip_graphs is False
  assert graphs._signature((torch.zeros(2),), {}) is None            # host tensors run eagerly
  assert graphs._signature((object(),), {}) is None                  # unsupported argument
  assert graphs._signature((1, None, True), {"b": 2.0, "a": "x"}) == (("a", "b"), (1, None, True, "x", 2.0))

  calls = []

  class Module:
    @graphs.graphed
    def forward(self, x, *, flag=False):
      calls.append(flag)
      return x

  config.configure_runtime(hip_graphs=True)
  m = Module()
  for _ in range(3):
    m.forward(torch.zeros(2), flag=True)
  assert calls == [True] * 3 and "_hip_graph_cache" not in m.__dict__


def test_transition_factories_are_replaced(reset_runtime):
  original_trunk, original_diff = M.TransitionBlock, M.DiffusionTransitionBlock
  config.configure_runtime(backend="hip", device="cuda",
                           native_ops=["evoformer_transition_block", "diffusion_transition_block"])
  backends.init()
  assert M.TransitionBlock.__name__ == "TransitionBlockHip" and issubclass(M.TransitionBlock, original_trunk)
  assert M.DiffusionTransitionBlock.__name__ == "DiffusionTransitionBlockHip"
  t = M.TransitionBlock(M.TransitionBlock.Config(), M.GlobalConfig(), num_channels=64)
  with pytest.raises(RuntimeError, match="not prepared"):
    t(torch.zeros(3, 64))
  config.configure_runtime(backend="torch")
  backends.init()
  assert M.TransitionBlock is original_trunk and M.DiffusionTransitionBlock is original_diff


def test_trimul_incoming_edge_is_read_from_either_equation_form():
  """The reference module keeps the per-channel einsum form (blocks.py:447-451); the config keeps
  the pair form.  Both name the incoming edge."""
  from sparsefold_amd.backends.hip import modules as HM
  inc = HM.TriangleMultiplicationHipMixin.INCOMING_EQUATIONS
  assert "...kjc,...kic->...ijc" in inc and "...ckj,...cki->...cij" in inc
  assert "...ikc,...jkc->...ijc" not in inc and "...cik,...cjk->...cij" not in inc


def test_sparse_attention_settings_and_parameters(monkeypatch, reset_runtime):
  """IBSAParameters.default reads the runtime's sparse_attention_parameters over the field
  defaults (blocks.py:405-418, runtime/config.py:27,68 of the reference)."""
  assert config.sparse_attention_parameters == {} and config.enable_gsa_index_reuse is True
  assert M.IBSAParameters.default() == M.IBSAParameters(16, 6, 0.90, 0.95, 0.02)
  monkeypatch.setenv("SPARSEFOLD_SPARSE_ATTENTION_PARAMETERS", "{'num_samples': 8, 'num_rand_blocks': 5}")
  config.reset()
  assert M.IBSAParameters.default() == M.IBSAParameters(8, 5, 0.90, 0.95, 0.02)
  config.configure_runtime(sparse_attention_parameters={"t_prob": 0.5}, hip_sparse_grid_attention=True)
  assert M.IBSAParameters.default().t_prob == 0.5 and config.hip_sparse_grid_attention is True
  opts = config.get_runtime_options()
  opts["sparse_attention_parameters"]["t_prob"] = 0.1
  assert config.sparse_attention_parameters["t_prob"] == 0.5
  with pytest.raises(ValueError, match="dict"):
    config.configure_runtime(sparse_attention_parameters="[1, 2]")


def test_index_reuser_follows_policy_and_switch(reset_runtime):
  reuser = M.IndexReuser(lambda idx: (0,) if idx == (2,) else None)
  reuser.set(0, "maps of layer 0")
  assert reuser.get((2,)) == ("maps of layer 0", (0,))
  assert reuser.get([1]) == (None, None)
  config.configure_runtime(enable_gsa_index_reuse=False)
  assert reuser.get((2,)) == (None, None)
  assert M.default_reuse_policy((3,)) is None


def test_grid_attention_takes_the_native_backends_sparse_arguments(reset_runtime):
  config.configure_runtime(backend="hip", device="cuda", native_ops=["grid_self_attn"])
  backends.init()
  p = M.IBSAParameters(num_samples=4)
  m = M.GridSelfAttention(M.GridSelfAttention.Config(), M.GlobalConfig(), True, num_channels=128,
                          ibsa_params=p, index_reuse_policy=M.default_reuse_policy)
  assert m.ibsa_params_provider((0,)) is p and m.index_reuse_policy is M.default_reuse_policy
  provider = lambda indices: M.IBSAParameters(num_samples=len(indices))
  m2 = M.GridSelfAttention(M.GridSelfAttention.Config(), M.GlobalConfig(), False, num_channels=128,
                           ibsa_params=provider)
  assert m2.ibsa_params_provider((0, 1)).num_samples == 2
  assert m2.ibsa_params_provider is provider
