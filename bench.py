"""Benchmark: triangle attention (starting node) at N=768 on one MI355X.

Workload (the headline configuration): z bf16 [768, 768, 128] ~ N(0,1), 4 heads x 32,
bias [4, 768, 768] from LN(z) W_b, sigmoid gate, output projection and residual -- one
call of GridSelfAttention.forward through the HIP backend.  A "step" is one such call with
z already resident in HBM.

Reports ms/call and the fraction of dense bf16 MFMA peak on the module's algorithmic FLOP
(4*H*D*N^3 attention + 2*N^2*C*(4*H*D + H) projections + 2*N^2*H*D*C output projection), a
roofline object for the dominant kernel (the attention core, timed live with HIP events on
the stream it runs on), and the host-CPU Torch math path (oracle restatement of the reference
composite in bf16, 128-row chunks) timed on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import torch

N, C, H, D = 768, 128, 4, 32
PEAK_BF16_TFLOPS = 2500.0          # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0
CLOCK_WARMUP_S = 0.5               # minimum wall time of untimed calls before the timed steps


def module_flop(n=N, c=C, h=H, d=D) -> float:
  attn = 4.0 * h * d * n ** 3
  proj = 2.0 * n * n * c * (4 * h * d + h)
  out = 2.0 * n * n * h * d * c
  return attn + proj + out


def core_flop(n=N, h=H, d=D) -> float:
  return 4.0 * h * d * n ** 3


def parse():
  ap = argparse.ArgumentParser()
  ap.add_argument("--gpus", type=int, default=1)
  ap.add_argument("--steps", type=int, default=200)
  ap.add_argument("--warmup", type=int, default=50, help="untimed calls first (the GPU clock ramps up)")
  ap.add_argument("--cpu-baseline", type=int, default=1, help="time the host-CPU math path (rank 0)")
  ap.add_argument("--other-configs", type=int, default=1, help="also time the other four configurations")
  ap.add_argument("--profile-config", default="",
                  help="only run this configuration --steps times (e.g. single_n768) and exit")
  ap.add_argument("--copy-mib", type=int, default=0,
                  help="only run a plain device-to-device copy of this many MiB 5 times and exit "
                       "(the known-size kernel that calibrates FETCH_SIZE / WRITE_SIZE counters)")
  return ap.parse_args()


def _events_time(fn, iters: int, stream) -> float:
  start = torch.cuda.Event(enable_timing=True)
  end = torch.cuda.Event(enable_timing=True)
  start.record(stream)
  for _ in range(iters):
    fn()
  end.record(stream)
  end.synchronize()
  return start.elapsed_time(end) / iters


def _median_call_ms(fn, iters: int, stream) -> float:
  """Median duration of single calls, each bracketed by its own pair of HIP events on `stream`
  (the rule for the parity configurations' timings; `value` stays the mean over a block of calls,
  as the step contract has it)."""
  pairs = []
  for _ in range(iters):
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    fn()
    e1.record(stream)
    pairs.append((e0, e1))
  torch.cuda.synchronize()
  times = sorted(e0.elapsed_time(e1) for e0, e1 in pairs)
  return times[len(times) // 2]


def stage_ms(z, seq, mod, iters: int) -> dict:
  """Average duration of each triangle stage (projection, attention core, output projection),
  launched through sf_hip_triangle_stage_fwd on the current stream and timed with HIP events
  recorded on that same stream."""
  from sparsefold_amd import _lib
  from sparsefold_amd.backends.hip import ops
  ws = torch.empty(ops.triangle_workspace_bytes(N, C, H, D), dtype=torch.uint8, device=z.device)
  out = torch.empty_like(z)
  args = (z, seq, mod._hip_ln_w, mod._hip_ln_b, mod._hip_w_qkvgb, mod._hip_w_o)
  kw = dict(num_head=H, transpose=False, workspace=ws, out=out)
  ops.triangle_attention(*args, **kw, stages=_lib.TRI_STAGE_ALL)
  torch.cuda.synchronize()
  res = {}
  for name, st in (("project", _lib.TRI_STAGE_PROJECT), ("attend", _lib.TRI_STAGE_ATTEND),
                   ("output", _lib.TRI_STAGE_OUTPUT)):
    res[name] = _events_time(lambda: ops.triangle_attention(*args, **kw, stages=st), iters,
                             torch.cuda.current_stream())
  return res


def copy_calibration(mib: int) -> None:
  """A plain copy of `mib` MiB: reads and writes exactly mib MiB of HBM per launch."""
  n = mib << 20
  src = torch.randint(0, 255, (n,), dtype=torch.uint8, device="cuda:0")
  dst = torch.empty_like(src)
  for _ in range(5):
    dst.copy_(src)
  torch.cuda.synchronize()
  print(json.dumps({"copy_mib": mib, "launches": 5, "bytes_read_per_launch": n, "bytes_written_per_launch": n}))


def traffic_from_profile() -> float | None:
  """HBM bytes per tri_attn_kernel launch, as recorded from the FETCH_SIZE / WRITE_SIZE counter
  runs (calibrated against a plain copy) in profiles/tri_attn_kernel_n768_traffic.md."""
  path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "tri_attn_kernel_n768_traffic.md")
  try:
    with open(path) as f:
      for line in f:
        if line.startswith("traffic_bytes_per_launch:"):
          return float(line.split(":", 1)[1])
  except OSError:
    return None
  return None


CONFIG_MIN_TIMED_S = 0.05           # minimum GPU time of a configuration's timed calls


def _time_call(fn, iters: int) -> float:
  """Mean ms of one call: the same clock warm-up as the headline (calls for at least
  CLOCK_WARMUP_S of wall time, then 20 more), then at least `iters` timed calls and at least
  CONFIG_MIN_TIMED_S of them, by HIP events on the current stream."""
  t0 = time.perf_counter()
  calls = 0
  while time.perf_counter() - t0 < CLOCK_WARMUP_S or calls < 20:
    fn()
    calls += 1
    if calls % 10 == 0:
      torch.cuda.synchronize()
  torch.cuda.synchronize()
  per_call_s = (time.perf_counter() - t0) / calls
  n = max(iters, int(CONFIG_MIN_TIMED_S / max(per_call_s, 1e-6)) + 1)
  return _events_time(fn, n, torch.cuda.current_stream())


def _config_builders(side_timings: bool = True) -> dict:
  """name -> builder() returning (call, metrics(t_ms) -> dict) for the remaining parity
  configurations, each one module call with inputs resident in HBM.  Algorithmic work: FLOP
  for the MFMA-bound forms, bytes for the HBM-bound ones."""
  from sparsefold_amd import backends
  from sparsefold_amd import workloads as W
  dev = torch.device("cuda:0")

  def c1():    # triangle attention, starting node, N=20, fp32 activations (launch-latency bound)
    mod, z, seq = W.make_triangle(20, dtype=torch.float32, seed=1)
    mod = mod.to(dev); backends.prepare(mod)
    z, seq = z.to(dev), seq.to(dev)
    return (lambda: mod(z, seq)), (lambda t: {"us_per_call": round(t * 1e3, 2), "bound": "latency"})

  def c2(tr):  # triangle attention N=384, starting / ending node, last N//10 tokens padded
    def build():
      mod, z, seq = W.make_triangle(384, padded=True, transpose=tr, seed=2)
      mod = mod.to(dev); backends.prepare(mod)
      z, seq = z.to(dev), seq.to(dev)
      f = module_flop(384)
      return (lambda: mod(z, seq)), (lambda t: {"ms_per_call": round(t, 4), "tflops": round(f / t / 1e9, 1),
                                                "frac_bf16_peak": round(f / t / 1e9 / PEAK_BF16_TFLOPS, 4),
                                                "bound": "mfma"})
    return build

  def c3b():   # single attention with pair bias, N=768 (pair-logit prologue reads z: HBM-bound)
    n, cs, cz, h, d = 768, 384, 128, 16, 24
    mod, z, s_act, seq = W.make_single(n, seed=3)
    mod = mod.to(dev); backends.prepare(mod)
    z, s_act, seq = z.to(dev), s_act.to(dev), seq.to(dev)
    bytes_ = n * n * cz * 2 + h * n * n * 2 + 2 * n * cs * 2            # z, bias planes once, s in/out
    flop = (2 * n * n * cz * h) + 2 * n * cs * 4 * cs + 4 * h * n * n * d + 2 * n * cs * cs
    return (lambda: mod(z, s_act, seq)), (lambda t: {
        "ms_per_call": round(t, 4), "gbs": round(bytes_ / t / 1e6, 1),
        "frac_hbm_peak": round(bytes_ / t / 1e6 / PEAK_HBM_GBS, 4), "tflops": round(flop / t / 1e9, 2),
        "bound": "hbm"})

  def c4():    # diffusion-transformer token attention, 5 samples x N=1024, one block
    S, n, c, sc, h, d = 5, 1024, 768, 384, 16, 48
    mod, act, cond, bias, mask = W.make_diffusion(n, S=S, seed=4)
    mod = mod.to(dev); backends.prepare(mod)
    act, cond, bias, mask = act.to(dev), cond.to(dev), bias.to(dev), mask.to(dev)
    flop = (2 * n * sc * 2 * c + 2 * S * n * c * 4 * c + 4 * h * n * n * d * S + 2 * S * n * c * c
            + 2 * n * sc * c)
    return (lambda: mod(act, mask, pair_logits=bias, single_cond=cond)), (lambda t: {
        "ms_per_call": round(t, 4), "ms_24_blocks": round(24 * t, 3), "tflops": round(flop / t / 1e9, 1),
        "frac_bf16_peak": round(flop / t / 1e9 / PEAK_BF16_TFLOPS, 4), "bound": "mfma"})

  def c4_stack():  # the 24 attention blocks of the diffusion Transformer, 5 samples x N=1024, each
    # with its own seeded weights: every block's AdaLN conditioning in one call, then the 24 blocks
    # on their precomputed layers (the transition blocks between them are timed separately)
    from sparsefold_amd.backends.hip import ops as HO
    S, n, c, sc, h, d, L = 5, 1024, 768, 384, 16, 48, 24
    mods, act, cond, bias, mask = W.make_diffusion_stack(n, S=S, L=L, seed=4)
    mods = [m.to(dev) for m in mods]
    for m in mods:
      backends.prepare(m)
    act, cond, bias, mask = act.to(dev), cond.to(dev), bias.to(dev), mask.to(dev)
    stacked = (torch.stack([m._hip_ada_lnc_w for m in mods]), torch.cat([m._hip_ada_w_scale for m in mods]),
               torch.cat([m._hip_ada_b_scale for m in mods]), torch.cat([m._hip_ada_w_shift for m in mods]),
               torch.cat([m._hip_w_zc for m in mods]), torch.cat([m._hip_b_zc for m in mods]))
    flop = L * (2 * n * sc * 2 * c + 2 * S * n * c * 4 * c + 4 * h * n * n * d * S + 2 * S * n * c * c
                + 2 * n * sc * c)

    def call():
      scale, shift, zgate = HO.diffusion_conditioning(cond, *stacked)
      x = act
      for layer, m in enumerate(mods):
        x = m(x, mask, pair_logits=bias, adaptive_scale=scale[layer], adaptive_bias=shift[layer],
              zero_gate=zgate[layer])
      return x
    return call, (lambda t: {
        "ms_per_block": round(t / L, 4), "ms_24_blocks": round(t, 3), "tflops": round(flop / t / 1e9, 1),
        "frac_bf16_peak": round(flop / t / 1e9 / PEAK_BF16_TFLOPS, 4), "bound": "mfma"})

  def c4_transition():  # diffusion-transformer transition block, 5 samples x N=1024, C=768, I=1536
    S, n, c, sc, inter = 5, 1024, 768, 384, 1536
    mod, act, cond = W.make_diffusion_transition(n, S=S, seed=11, sharp=False)
    mod = mod.to(dev); backends.prepare(mod)
    act, cond = act.to(dev), cond.to(dev)
    flop = 2 * S * n * c * 2 * inter + 2 * S * n * inter * c + 2 * n * sc * 3 * c
    return (lambda: mod(act, single_cond=cond)), (lambda t: {
        "ms_per_call": round(t, 4), "tflops": round(flop / t / 1e9, 1),
        "frac_bf16_peak": round(flop / t / 1e9 / PEAK_BF16_TFLOPS, 4), "bound": "mfma"})

  def trunk_transition(n_rows, c, lead):  # trunk transition: single (C=384) or pair (C=128), I = 4C
    def build():
      mod, act = W.make_transition(n_rows, C=c, lead=lead, seed=12, sharp=False)
      mod = mod.to(dev); backends.prepare(mod)
      act = act.to(dev)
      rows = act.numel() // c
      flop = 2 * rows * c * 8 * c + 2 * rows * 4 * c * c
      return (lambda: mod(act)), (lambda t: {
          "ms_per_call": round(t, 4), "tflops": round(flop / t / 1e9, 1),
          "frac_bf16_peak": round(flop / t / 1e9 / PEAK_BF16_TFLOPS, 4), "bound": "mfma"})
    return build

  def trimul(n, incoming):  # triangle multiplicative update, z [n, n, 128], outgoing / incoming edges
    def build():
      mod, z, mask = W.make_trimul(n, incoming=incoming, padded=True, seed=13, sharp=False)
      mod = mod.to(dev); backends.prepare(mod)
      z, mask = z.to(dev), mask.to(dev)
      c = 128
      flop = 2 * n ** 3 * c + 2 * n * n * c * 4 * c + 2 * n * n * c * 2 * c
      return (lambda: mod(z, mask)), (lambda t: {
          "ms_per_call": round(t, 4), "tflops": round(flop / t / 1e9, 1),
          "frac_bf16_peak": round(flop / t / 1e9 / PEAK_BF16_TFLOPS, 4), "bound": "mfma"})
    return build

  def c5():    # windowed atom attention, 5 samples x 8192 atoms, 32-query / 128-key windows
    # The keys' condition is the gathered queries' (as CrossAttTransformer builds it), so the call
    # is the per-atom plan: both sides' AdaLN terms once per example (cached by the module, as the
    # native reference caches them), K/V per atom, windows gathered inside the attention.
    # `ms_per_call_general`: the same inputs with the key condition given per window key.
    S, atoms, c, h, d = 5, 8192, 128, 4, 32
    mod, act, lay, qc, kc, bias = W.make_window(atoms, S=S, seed=5)
    mod = mod.to(dev); backends.prepare(mod)
    act, qm, gi, gm, km, qc, kc, bias = (x.to(dev) for x in (act, lay.queries_mask, lay.gather_idxs, lay.gather_mask,
                                                            lay.keys_mask, qc, kc, bias))
    U = atoms // 32
    flop = 4 * h * 32 * 128 * d * U * S + 2 * S * atoms * c * 2 * c * 2 + 2 * S * atoms * c * c
    bytes_ = 2 * S * atoms * c * 2 + U * h * 32 * 128 * 2 + (atoms + U * 128) * c * 2
    general_ms = _time_call(lambda: mod.forward_indexed(act, qm, gi, gm, km, qc, kc, bias), 20) if side_timings else None
    return (lambda: mod.forward_indexed(act, qm, gi, gm, km, qc, None, bias)), (lambda t: {
        "ms_per_call": round(t, 4), "ms_per_call_general": general_ms and round(general_ms, 4),
        "tflops": round(flop / t / 1e9, 2), "gbs": round(bytes_ / t / 1e6, 1),
        "frac_bf16_peak": round(flop / t / 1e9 / PEAK_BF16_TFLOPS, 4),
        "frac_hbm_peak": round(bytes_ / t / 1e6 / PEAK_HBM_GBS, 4), "bound": "balanced"})

  def pack_tr():  # diffusion Transformer pair-logit pack, N=1024: [1024,1024,128] -> [6,4,16,1024,1024]
    n, pc, planes = 1024, 128, 384
    mod, pair_cond = W.make_transformer_pack(n, seed=6)
    mod = mod.to(dev); backends.prepare(mod)
    pair_cond = pair_cond.to(dev)
    bytes_ = n * n * pc * 2 + planes * n * n * 2
    return (lambda: mod.pair_logits_pack(pair_cond)), (lambda t: {
        "ms_per_call": round(t, 4), "gbs": round(bytes_ / t / 1e6, 1),
        "frac_hbm_peak": round(bytes_ / t / 1e6 / PEAK_HBM_GBS, 4), "bound": "hbm"})

  def pack_x():  # atom CrossAttTransformer pack, 8192 atoms: [256,32,128,16] -> [3,256,4,32,128]
    U, pc, planes = 256, 16, 12
    mod, pair_cond = W.make_cross_pack(U, seed=8)
    mod = mod.to(dev); backends.prepare(mod)
    pair_cond = pair_cond.to(dev)
    bytes_ = U * 32 * 128 * (pc + planes) * 2
    return (lambda: mod.pair_logits_pack(pair_cond)), (lambda t: {
        "ms_per_call": round(t, 4), "gbs": round(bytes_ / t / 1e6, 1),
        "frac_hbm_peak": round(bytes_ / t / 1e6 / PEAK_HBM_GBS, 4), "bound": "hbm"})

  def dense(n, padded=False, c=C):  # triangle attention, starting node; all-ones mask (the block-sparse
    # lines' baseline), or the last n//10 tokens padded; c=64: the template stack's shape (H=4, D=16)
    def build():
      mod, z, seq = W.make_triangle(n, C=c, H=4, seed=9, padded=padded)
      mod = mod.to(dev); backends.prepare(mod)
      z, seq = z.to(dev), seq.to(dev)
      f = module_flop(n, c, 4, c // 4)
      return (lambda: mod(z, seq)), (lambda t: {"ms_per_call": round(t, 4), "tflops": round(f / t / 1e9, 1),
                                                "frac_bf16_peak": round(f / t / 1e9 / PEAK_BF16_TFLOPS, 4),
                                                "bound": "mfma"})
    return build

  def ibs(n):  # block-sparse (IBS) triangle attention, starting node, default parameters
    # (num_samples 16, num_rand_blocks 5, t_prob 0.9, tr_prob 0.95, u_prob 0.02): maps sampled on
    # every call; `ms_per_call_reuse` reuses them (a later layer under an index-reuse policy)
    from sparsefold_amd.backends.hip import ops as HO
    def build():
      mod, z, seq = W.make_triangle(n, seed=9)
      mod = mod.to(dev); backends.prepare(mod)
      z, seq = z.to(dev), seq.to(dev)
      ws = torch.empty(HO.triangle_ibs_workspace_bytes(n, 128, 4, 32), dtype=torch.uint8, device=dev)
      out = torch.empty_like(z)
      kw = dict(num_head=4, transpose=False, num_samples=16, num_rand_blocks=5, t_prob=0.9, tr_prob=0.95,
                u_prob=0.02, workspace=ws, out=out)
      args = (z, seq, mod._hip_ln_w, mod._hip_ln_b, mod._hip_w_qkvgb, mod._hip_w_o)
      _, im, wm = HO.triangle_attention_ibs(*args, seed=1, **kw)
      frac = float((im >= 0).sum()) / (im.numel() / 16 * ((n + 31) // 32))
      reuse_ms = _time_call(lambda: HO.triangle_attention_ibs(*args, index_map=im, weight_map=wm, **kw), 20) \
          if side_timings else None
      return (lambda: HO.triangle_attention_ibs(*args, seed=1, **kw)), (lambda t: {
          "ms_per_call": round(t, 4), "ms_per_call_reuse": reuse_ms and round(reuse_ms, 4),
          "key_blocks_attended": round(frac, 3), "bound": "mfma"})
    return build

  return {"triangle_n20_fp32": c1, "triangle_n384_start": c2(False), "triangle_n384_end": c2(True),
          "triangle_n768_padded": dense(768, padded=True), "triangle_template_n768": dense(768, c=64),
          "triangle_ibs_n768": ibs(768), "triangle_n1536_start": dense(1536), "triangle_ibs_n1536": ibs(1536),
          "single_n768": c3b, "diffusion_5x1024_block": c4,
          "diffusion_5x1024_24_blocks": c4_stack, "diffusion_transition_5x1024": c4_transition,
          "single_transition_n768": trunk_transition(768, 384, ()),
          "pair_transition_n384": trunk_transition(384, 128, (384,)),
          "trimul_outgoing_n768": trimul(768, False), "trimul_incoming_n768": trimul(768, True),
          "window_5x8192": c5,
          "transformer_pack_n1024": pack_tr, "cross_pack_8192": pack_x}


def other_configs(iters: int) -> dict:
  """Times every configuration of _config_builders (median-free: HIP events over `iters`
  calls after a warm-up).  The module configurations are timed twice: eagerly (the line's
  numbers) and with HIP-graph replay of the repeated call (`ms_per_call_hip_graphs`; the same
  kernels, one graph launch instead of one launch per kernel)."""
  from sparsefold_amd.runtime import config
  res = {}
  for name, build in _config_builders().items():
    call, metrics = build()
    res[name] = metrics(_time_call(call, iters if "24_blocks" not in name else max(iters // 8, 5)))
    if "pack" not in name and "24_blocks" not in name and "ibs" not in name:
      config.configure_runtime(backend="hip", sdpa_implementation="hip", device="cuda", hip_graphs=True)
      try:
        res[name]["ms_per_call_hip_graphs"] = round(_time_call(call, iters), 4)
      finally:
        config.configure_runtime(backend="hip", sdpa_implementation="hip", device="cuda")
  return res


def profile_config(name: str, calls: int) -> None:
  """Runs one configuration `calls` times (for rocprofv3 kernel statistics); the builders' side
  timings (the general window path, map reuse) are skipped, so the trace holds this call only."""
  builders = _config_builders(side_timings=False)
  if name not in builders:
    raise SystemExit(f"unknown configuration {name!r}; one of {sorted(builders)}")
  call, _ = builders[name]()
  for _ in range(calls):
    call()
  torch.cuda.synchronize()
  print(f"[bench] profiled {name}: {calls} calls", flush=True)


def _host_cpu() -> dict:
  """The host CPU as the baseline protocol asks: model, physical cores of the affinity set,
  affinity set size and AMX-BF16 presence (from /proc/cpuinfo and the sysfs topology)."""
  aff = sorted(os.sched_getaffinity(0))
  model, flags = "unknown", set()
  try:
    with open("/proc/cpuinfo") as f:
      for line in f:
        if line.startswith("model name") and model == "unknown":
          model = line.split(":", 1)[1].strip()
        elif line.startswith("flags") and not flags:
          flags = set(line.split(":", 1)[1].split())
  except OSError:
    pass
  cores = set()
  for cpu in aff:
    base = f"/sys/devices/system/cpu/cpu{cpu}/topology/"
    try:
      with open(base + "physical_package_id") as f1, open(base + "core_id") as f2:
        cores.add((f1.read().strip(), f2.read().strip()))
    except OSError:
      cores.add(("?", str(cpu)))
  return {"cpu_model": model, "physical_cores": len(cores), "affinity_cpus": len(aff),
          "amx_bf16": "amx_bf16" in flags}


def cpu_baseline() -> dict:
  """Host-CPU Torch math path: the oracle restatement of GridSelfAttention.forward
  (blocks.py:293-366) in bf16 with SDPA MATH and 128-row chunks (configs/cpu.toml: sdpa "math",
  runtime.sharding), on the same seeded inputs as the GPU measurement, under
  torch.inference_mode with one thread per physical core of the affinity set.  The whole call
  (all 768 rows) is timed: median of 5 runs after 2 warm-ups."""
  from oracle import modules as OM
  from sparsefold_amd import workloads as W
  host = _host_cpu()
  threads = max(1, host["physical_cores"])
  torch.set_num_threads(threads)
  mod, z, seq = W.make_triangle(N, seed=3)
  p = {k: v.to(torch.bfloat16) for k, v in W.state_dict_f32(mod).items()}
  times = []
  with torch.inference_mode():
    for i in range(7):
      t0 = time.perf_counter()
      OM.grid_self_attention(z, seq, p, transpose=False, chunk_size=128)
      times.append(time.perf_counter() - t0)
      print(f"[bench]   cpu run {i} ({'warm-up' if i < 2 else 'timed'}): {times[-1]:.2f} s", flush=True)
  timed = sorted(times[2:])
  med = timed[len(timed) // 2]
  return {"value": med * 1e3, "unit": "ms/call", "cores": threads, "kind": "port",
          "sample": f"the whole N=768 call (prologue + all {N} rows in 128-row chunks), bf16 Torch math "
                    "(oracle restatement of blocks.py:293-366, SDPA MATH); median of 5 after 2 warm-ups",
          "runs_s": [round(t, 3) for t in times], **host}


def main():
  args = parse()
  if args.gpus != 1:
    print(json.dumps({"error": "this build runs on one GPU; multi-GPU sharding is a design note only",
                      "n_gpus": args.gpus}))
    sys.exit(2)
  if args.copy_mib:
    copy_calibration(args.copy_mib)
    return
  if args.profile_config:
    from sparsefold_amd import backends
    from sparsefold_amd.runtime import config
    config.configure_runtime(backend="hip", sdpa_implementation="hip", device="cuda")
    backends.init()
    profile_config(args.profile_config, args.steps)
    return
  from sparsefold_amd import backends
  from sparsefold_amd import workloads as W
  from sparsefold_amd.runtime import config

  config.configure_runtime(backend="hip", sdpa_implementation="hip", device="cuda")
  backends.init()
  dev = torch.device("cuda:0")
  mod, z, seq = W.make_triangle(N, seed=3)
  mod = mod.to(dev)
  backends.prepare(mod)
  z, seq = z.to(dev), seq.to(dev)
  stream = torch.cuda.current_stream()
  print(f"[bench] triangle start N={N} C={C} H={H} D={D} warmup={args.warmup} steps={args.steps}", flush=True)
  # the GPU clock ramps up under load: besides the W warm-up calls, calls run until at least
  # CLOCK_WARMUP_S of wall time has passed, whatever W is, so that short runs time a steady clock
  t0 = time.perf_counter()
  extra = 0
  while time.perf_counter() - t0 < CLOCK_WARMUP_S:
    for _ in range(10):
      mod(z, seq)
    torch.cuda.synchronize()
    extra += 10
  for _ in range(args.warmup):
    mod(z, seq)
  torch.cuda.synchronize()
  ms = _events_time(lambda: mod(z, seq), args.steps, stream)
  torch.cuda.synchronize()
  median_ms = _median_call_ms(lambda: mod(z, seq), max(args.steps, 20), stream)
  stages = stage_ms(z, seq, mod, max(args.steps, 10))
  core_ms = stages["attend"]
  flop = module_flop()
  tflops = flop / (ms * 1e-3) / 1e12
  core_tflops = core_flop() / (core_ms * 1e-3) / 1e12
  print(f"[bench] module {ms:.3f} ms ({tflops:.1f} TFLOP/s); stages "
        + ", ".join(f"{k} {v:.3f} ms" for k, v in stages.items())
        + f"; attention core {core_tflops:.1f} TFLOP/s", flush=True)
  others = None
  if args.other_configs:
    print("[bench] timing the other configurations...", flush=True)
    others = other_configs(max(args.steps // 2, 5))
    for k, v in others.items():
      print(f"[bench]   {k}: {v}", flush=True)
  cpu = None
  if args.cpu_baseline:
    print("[bench] timing host-CPU math path sample...", flush=True)
    cpu = cpu_baseline()
    print(f"[bench] cpu baseline {cpu['value']:.1f} ms/call on {cpu['cores']} threads", flush=True)
  line = {
      "metric": "ms/call + % bf16 MFMA peak, triangle attention N=768; vs host-CPU math path",
      "value": round(ms, 4),
      "unit": "ms/call",
      "n_gpus": 1,
      "steps": args.steps,
      "warmup": args.warmup,
      "clock_warmup": {"calls": extra, "min_seconds": CLOCK_WARMUP_S},
      "ms_per_step": round(ms, 4),
      "ms_per_call_median": round(median_ms, 4),
      "higher_is_better": False,
      "scaling": "weak",
      "vs_baseline": None,
      "dtype": "bf16",
      "data": "synthetic (seeded N(0,1) z, N(0,0.02^2) weights)",
      "config": {"workload": "triangle attention, starting node, N=768, C=128, H=4, D=32, all-ones mask",
                 "module_flop": flop, "tflops": round(tflops, 2),
                 "pct_bf16_peak": round(100 * tflops / PEAK_BF16_TFLOPS, 2)},
      "stages_ms": {k: round(v, 4) for k, v in stages.items()},
      "roofline": {"bound": "mfma", "kernel": "tri_attn_kernel", "achieved": round(core_tflops, 2),
                   "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(core_tflops / PEAK_BF16_TFLOPS, 4),
                   "traffic": traffic_from_profile(), "kernel_ms": round(core_ms, 4), "flop_per_launch": core_flop()},
      "other_configs": others,
      "cpu_baseline": cpu,
      "speedup_vs_cpu": None if cpu is None else round(cpu["value"] / ms, 1),
  }
  print(json.dumps(line), flush=True)


if __name__ == "__main__":
  main()
