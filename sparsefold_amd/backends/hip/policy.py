"""Selection checks for the HIP backend (mirrors ``backends/vecops/policy.py:15-42``)."""
from collections.abc import Sequence

# native.ops names (src/sparsefold/config.py:24-35) that this backend replaces
HIP_NATIVE_OPS = frozenset({
    "grid_self_attn", "evoformer_single_act_update", "diffusion_self_attention", "diffusion_cross_attention",
    "evoformer_transition_block", "diffusion_transition_block", "triangle_multiplication",
})
# names the reference accepts that are outside the attention path: accepted, left on Torch
OTHER_NATIVE_OPS = frozenset({"linear", "msa_attention", "outer_product_mean"})


def validate_hip_device(device) -> None:
  if str(device).split(":", 1)[0] not in {"cuda", "hip"}:
    raise RuntimeError("HIP kernels run on the GPU only; configure device='cuda'")


def validate_hip_ops(selected: Sequence[str]) -> None:
  chosen = set(selected)
  if chosen & {"*", "all"}:
    return
  unknown = chosen - HIP_NATIVE_OPS - OTHER_NATIVE_OPS
  if unknown:
    raise ValueError(f"Unknown native operators: {sorted(unknown)}")
