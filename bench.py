"""Throughput of the batched Junqi env-step on one MI355X.

One step = for every game: draw an action uniformly from its legal row
(Philox4x32-10), apply the ply, auto-reset finished games from the setup pool,
generate the next acting seat's legal actions (sorted CSR + packed canonical
mask) and its 317-plane observation (u8 codes + aux rows + 28 globals).
Prints one JSON line. Usage: python bench.py [--steps K] [--warmup W] [--envs N]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
OBS_U8_BYTES = 317 * 289          # 91,613
AUX_BYTES = 8 + 4 * 289 * 2       # 2,320: turn history f32[2] + recency codes u16[4][289]
GLOBAL_BYTES = 28 * 4             # 112
MASK_BYTES = 521 * 4              # 2,084


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--envs", type=int, default=32768)
    ap.add_argument("--fmt", default="u8", choices=["u8", "bf16", "f32"])
    ap.add_argument("--path", default="fused", choices=["fused", "separate"],
                    help="fused: jq_env_step; separate: the same step through jq_sample_uniform, jq_step, "
                         "jq_reset_terminated and jq_legal, the reference collector's call order")
    ap.add_argument("--seed", type=int, default=0x4A51)
    ap.add_argument("--cpu-envs", type=int, default=4096)
    ap.add_argument("--cpu-steps", type=int, default=40)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MB",
                    help="only run a plain device copy of MB megabytes (counter calibration) and exit")
    return ap.parse_args()


def calibrate_copy(mb: int) -> int:
    """A plain device-to-device copy of known size, so hardware byte counters
    (FETCH_SIZE / WRITE_SIZE) can be scaled against it."""
    import torch

    n = mb * (1 << 20)
    a = torch.ones(n, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes": n, "launches": 3}), flush=True)
    return 0


def cpu_baseline(envs: int, steps: int) -> dict:
    """The C oracle (a scalar port, OpenMP over games) on this host's cores, on a
    bounded sample of the same workload: step + sorted legal ids + canonical mask
    + float32 observation of the acting seat."""
    import numpy as np

    from oracle import oracle as O

    setups = np.stack([O.random_setup(i) for i in range(envs)])
    batch = O.Batch(setups, show_mode=2)
    sp = np.zeros((envs, 317, 17, 17), np.float32)
    gl = np.zeros((envs, 28), np.float32)
    mask = np.zeros((envs, 2081), np.uint8)
    rng = np.random.default_rng(0)
    none = np.full(envs, -1, np.int32)
    batch.env_step(none, obs=True, mask_bits=mask, obs_spatial=sp, obs_global=gl)

    def pick():
        acts = np.full(envs, -1, np.int32)
        for i in range(envs):
            g = batch.games[i]
            if g["terminated"]:
                continue
            # any legal action will do for timing; use the oracle's own generator
            ids = np.zeros(4096, np.int32)
            n = O.lib().jqo_legal_ids(batch.games[i:i + 1].ctypes.data, int(g["turn"]), ids.ctypes.data, 4096)
            if n > 0:
                acts[i] = ids[rng.integers(n)]
        return acts

    total = 0.0
    for _ in range(steps):
        acts = pick()
        t0 = time.perf_counter()
        batch.env_step(acts, obs=True, mask_bits=mask, obs_spatial=sp, obs_global=gl)
        total += time.perf_counter() - t0
    return {"value": round(envs * steps / total, 1), "unit": "env-steps/s", "cores": O.omp_threads(),
            "kind": "port",
            "sample": f"{envs} games x {steps} env-steps (step + legal ids + canonical mask + f32 obs), "
                      f"random legal actions, HALF_DARK"}


# device kernel that writes the observation rows, per output format
OBS_KERNEL = {"f32": "jq::k_observe<0>", "bf16": "jq::k_observe<1>", "u8": "jq::k_observe_u8_persist"}


def measured_traffic(kernel: str, games: int):
    """HBM bytes per launch of `kernel` (FETCH_SIZE + WRITE_SIZE, scaled against a
    plain copy) from the committed counter summary, when it was taken at this size."""
    path = ROOT / "profiles" / "traffic.json"
    if games != 32768 or not path.exists():
        return None
    rec = json.loads(path.read_text()).get("kernels", {}).get(kernel)
    if not rec:
        return None
    return round(rec["read_bytes"] + rec["write_bytes"])


def main() -> int:
    args = parse()
    if args.calibrate_copy:
        return calibrate_copy(args.calibrate_copy)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the environment shards by games with no exchange "
              "(G GPUs = G independent batches), so it has no multi-GPU run", file=sys.stderr)
        return 2
    import numpy as np
    import torch

    import junqi_amd
    from junqi_amd import _lib as L

    n = args.envs
    b = junqi_amd.JunqiBatch(n, show_mode=2, max_num_moves=4000, pool_size=10000)
    dev = b.device
    b.reset(0)
    b.legal()
    es = {"u8": 1, "bf16": 2, "f32": 4}[args.fmt]
    sdt = {"u8": torch.uint8, "bf16": torch.bfloat16, "f32": torch.float32}[args.fmt]
    spatial = torch.empty((n, 317, 17, 17), dtype=sdt, device=dev)
    aux = torch.empty((n, AUX_BYTES), dtype=torch.uint8, device=dev) if args.fmt == "u8" else None
    glob = torch.empty((n, 28), dtype=torch.float32, device=dev)
    term = torch.empty(n, dtype=torch.uint8, device=dev)
    reward = torch.empty(n, dtype=torch.float32, device=dev)
    acts = torch.empty(n, dtype=torch.int32, device=dev)
    fmt_code = {"u8": L.OBS_U8, "bf16": L.OBS_BF16, "f32": L.OBS_F32}[args.fmt]
    h = b._h
    lib = L.lib
    P = lambda t: None if t is None else t.data_ptr()  # noqa: E731

    def one_step(ply: int, ev_obs=None):
        s = torch.cuda.current_stream(dev).cuda_stream
        # Philox pick from the previous CSR rows, ply, restart from the pool,
        # next seat's sorted CSR + packed canonical mask (jq_env_step without
        # the observation, which is launched on its own so events can time it)
        if args.path == "fused":
            L.check(lib.jq_env_step(h, None, L.SAMPLE_UNIFORM, args.seed, ply, ply, b.counts.data_ptr(),
                                    b.offsets.data_ptr(), b.values.data_ptr(), b.values.numel(),
                                    b.mask_words.data_ptr(), fmt_code, None, None, None, term.data_ptr(),
                                    reward.data_ptr(), None, acts.data_ptr(), s))
        else:
            L.check(lib.jq_sample_uniform(h, b.counts.data_ptr(), b.offsets.data_ptr(), b.values.data_ptr(),
                                          b.values.numel(), args.seed, ply, acts.data_ptr(), s))
            L.check(lib.jq_step(h, acts.data_ptr(), None, L.ACT_WORLD, None, None, term.data_ptr(), None, None,
                                None, None, reward.data_ptr(), None, s))
            L.check(lib.jq_reset_terminated(h, ply, s))
            L.check(lib.jq_legal(h, None, b.counts.data_ptr(), b.offsets.data_ptr(), b.values.data_ptr(),
                                 b.values.numel(), b.mask_words.data_ptr(), None, s))
        if ev_obs is not None:
            ev_obs[0].record()
        L.check(lib.jq_observe(h, None, fmt_code, 0, spatial.data_ptr(), P(aux), glob.data_ptr(), s))
        if ev_obs is not None:
            ev_obs[1].record()

    for w in range(args.warmup):
        one_step(w)
    torch.cuda.synchronize(dev)
    obs_events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(args.steps)]
    t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(dev)
    wall0 = time.perf_counter()
    t_start.record()
    for k in range(args.steps):
        one_step(args.warmup + k, obs_events[k])
    t_end.record()
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - wall0
    ms_total = t_start.elapsed_time(t_end)
    obs_ms = sum(a.elapsed_time(c) for a, c in obs_events) / args.steps
    legal_total = int(b.offsets[-1].item())

    steps_per_s = n * args.steps / (ms_total / 1e3)
    obs_bytes = n * (OBS_U8_BYTES * es + (AUX_BYTES if args.fmt == "u8" else 0) + GLOBAL_BYTES)
    achieved = obs_bytes / (obs_ms / 1e3) / 1e9
    kbar = legal_total / n
    rec = {
        "metric": "env-steps/sec incl. legal mask + obs at 32768 games on 1 MI355X; % HBM peak",
        "value": round(steps_per_s, 1),
        "unit": "env-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_total / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8" if args.fmt == "u8" else args.fmt,
        "data": "synthetic: seeded random legal setups, Philox-uniform legal actions, auto-reset from a 10000-setup pool",
        "config": {"workload": f"step + sorted legal CSR + packed canonical mask + 317-plane {args.fmt} obs "
                               f"of the acting seat, {n} games, HALF_DARK", "games": n, "obs_format": args.fmt,
                   "path": args.path,
                   "mean_legal_actions": round(kbar, 2)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(OBS_KERNEL[args.fmt], n),
                     "kernel": OBS_KERNEL[args.fmt], "kernel_ms": round(obs_ms, 4),
                     "bytes_per_launch": obs_bytes},
        "wall_s": round(wall, 3),
    }
    if not args.no_cpu:
        rec["cpu_baseline"] = cpu_baseline(args.cpu_envs, args.cpu_steps)
    print(json.dumps(rec), flush=True)
    b.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
