"""CPU oracle for SparseFold's gated pair-biased attention (TEST INFRASTRUCTURE).

This package is the checker, never the product.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only to compute expected values or to time the reference's CPU
math path.  The HIP path in ``sparsefold_amd`` never imports, links or falls
back to anything here.

Contents
--------
``sdpa``        restatement of ``dot_product_attention``
                (``src/sparsefold/backends/torch/attention/sdpa.py:22-121``).
``primitives``  ``Linear`` einsum conventions, ``LayerNorm`` and the CPU
                bounded sigmoid (``src/sparsefold/model/layers/primitives.py``).
``modules``     the four attention composites: triangle attention
                (``src/sparsefold/model/trunk/blocks.py:188-366``), single
                attention with pair bias (``blocks.py:692-763``,
                ``src/sparsefold/model/diffusion/transformer.py:234-345``),
                diffusion-transformer token attention (``transformer.py:348-477``)
                and windowed atom attention (``transformer.py:480-693`` with
                ``src/sparsefold/schema/atom_layout.py:52-83``).
``brute``       float64 numpy loop implementations used only to pin the
                restatement on tiny inputs (an implementation that shares no
                code with torch's SDPA).

How each function is pinned (every function has at least one check in
``tests/test_oracle_*.py``):

* ``sdpa.dot_product_attention`` -- against the float64 brute force, against
  ``torch.nn.functional.scaled_dot_product_attention`` (MATH) with the
  reference test's explicit additive mask (seed 808 shapes of
  ``tests/test_runtime_reference.py:117-138``), and known answers: fully masked
  row = mean of V over all keys, ``q=k=v=1`` -> ``q``
  (``tests/test_runtime_reference.py:141-145``), single key -> v, zero logits
  -> uniform mean.
* ``primitives.cpu_bounded_sigmoid`` -- closed form vs ``torch.sigmoid`` and
  the saturation limits; ``layer_norm`` vs a float64 numpy LN.
* ``modules.grid_self_attention`` -- float64 brute force at N<=6, the
  ending-node identity (end(z) == start(z^T) with the bias taken from the
  untransposed activations, transposed back), row-chunk independence, zero
  output projection -> identity.
* ``modules.self_attention`` / ``single_act_update`` -- float64 brute force,
  AdaLN-without-condition == LN, zero-init gate.
* ``modules.cross_attention`` / ``atom_layout_convert`` /
  ``windowed_cross_attention`` -- the reference's ``convert`` known answers
  (``tests/test_schema.py:76-86,187-196``, committed under
  ``tests/golden/``), windowed == dense masked attention over gathered keys.
"""
