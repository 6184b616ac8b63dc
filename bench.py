"""Throughput of the batched Junqi env-step on one MI355X.

One env-step = for every game: draw an action (masked N(0,1)-logit argmax over
the legal canonical ids, Philox4x32-10), apply the ply, restart a finished game
from the setup pool, generate the next acting seat's legal actions (sorted CSR
+ packed canonical mask) and its 317-plane observation (u8 codes + aux row +
28 globals), and record reward, done and Zobrist hash. That is the rollout loop
of the 32,768-game configuration; before timing, the batch is played into mixed
stages (game i starts S_i steps late, S_i uniform below --stagger), so the
timed window holds openings, middle games and endgames, and games end and
restart inside it.

Prints one JSON line. Usage: python bench.py [--steps K] [--warmup W]
  --config c5 (default): 32,768 games, logits sampler, step + CSR + mask + u8 obs;
      the line's "dropin" object times the same workload a second time through
      the reference collector's unchanged calls (f32 obs + bool mask; --no-dropin
      skips it)
  --config c3: 16,384 games at plies 0-400, uniform sampler, step + CSR + mask + obs
  --config c2: 4,096 games, uniform sampler, step + CSR + mask (no observation)
  --path fused | separate | dropin (the reference collector's GpuRollout calls)
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
OBS_ELEMS = 317 * 289             # 91,613 elements per observation
AUX_BYTES = 8 + 4 * 289 * 2       # 2,320: turn history f32[2] + recency codes u16[4][289]
GLOBAL_BYTES = 28 * 4             # 112
MASK_BYTES = 521 * 4              # 2,084 packed canonical mask
STEP_OUT_BYTES = 1 + 4 + 8 + 4    # terminated, reward, hash, action per env
METRIC = "env-steps/sec incl. legal mask + obs at 32768 games on 1 MI355X; % HBM peak"
CONFIGS = {
    "c5": dict(envs=32768, sampler="logits", obs=True, stagger=800),
    "c3": dict(envs=16384, sampler="uniform", obs=True, stagger=401),
    "c2": dict(envs=4096, sampler="uniform", obs=False, stagger=800),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c5", choices=sorted(CONFIGS))
    ap.add_argument("--envs", type=int, default=0, help="override the config's game count")
    ap.add_argument("--fmt", default="u8", choices=["u8", "bf16", "f32"])
    ap.add_argument("--sampler", default="", choices=["", "logits", "uniform"])
    ap.add_argument("--stagger", type=int, default=-1, help="mixed-stage warm-up steps (0 = all games fresh)")
    ap.add_argument("--show-mode", type=int, default=2, choices=[0, 1, 2])
    ap.add_argument("--path", default="fused", choices=["fused", "separate", "dropin"],
                    help="fused: jq_env_step; separate: jq_sample_* + jq_step + jq_reset_terminated + jq_legal; "
                         "dropin: GpuRollout's f32 observation, bool mask, canonical step and device reset")
    ap.add_argument("--seed", type=int, default=0x4A51)
    ap.add_argument("--cpu-envs", type=int, default=4096)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-dropin", action="store_true",
                    help="c5 fused only: skip the second timed run through GpuRollout's calls")
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


def fill_rate_gbps(nbytes: int, reps: int = 5) -> float:
    """Best write rate of a plain device fill of `nbytes` (torch's fill kernel
    on the current stream, timed with events): the practical ceiling of a
    kernel that only writes, measured on the same device."""
    import torch

    buf = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    for _ in range(2):
        buf.fill_(1)
    best = float("inf")
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        buf.fill_(2)
        e1.record()
        e1.synchronize()
        best = min(best, e0.elapsed_time(e1))
    del buf
    torch.cuda.empty_cache()
    return nbytes / (best / 1e3) / 1e9


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(envs: int, seconds: float, sampler: int, obs: bool, seed: int) -> dict:
    """The C oracle (a scalar port, OpenMP over games) on this host's cores, on a
    bounded sample of the same workload: sample -> step -> pool restart -> sorted
    legal ids + canonical mask (+ float32 observation of the acting seat), games
    first played into mixed stages. Timed for at least `seconds` on every host
    thread (`envs` games), then for at least 0.8 x `seconds` on one thread
    (envs / 4 games)."""
    import numpy as np

    from oracle import oracle as O

    pool = O.setup_pool(42, 1000)
    all_threads = O.omp_threads()

    def timed(n: int, target: float) -> tuple[float, int]:
        env = O.CpuEnv(np.stack([O.random_setup(i) for i in range(n)]), pool)
        for k in range(64):   # leave the opening: games spread over plies 0-64
            env.step(k, sampler=sampler, seed=seed, obs=False)
        env.step(64, sampler=sampler, seed=seed, obs=obs)   # first touch of the output pages
        t0, k = time.perf_counter(), 0
        while True:
            env.step(65 + k, sampler=sampler, seed=seed, obs=obs)
            k += 1
            el = time.perf_counter() - t0
            if el >= target:
                return n * k / el, k

    v_all, k_all = timed(envs, seconds)
    O.set_threads(1)
    n_one = max(1, envs // 4)
    v_one, k_one = timed(n_one, 0.8 * seconds)
    O.set_threads(all_threads)
    work = "step + sorted legal ids + canonical mask" + (" + f32 obs" if obs else "")
    return {"value": round(v_all, 1), "unit": "env-steps/s", "cores": all_threads, "kind": "port",
            "single_core_value": round(v_one, 1), "cpu_model": cpu_model(),
            "sample": f"{envs} games x {k_all} env-steps on {all_threads} threads and {n_one} x {k_one} on 1 "
                      f"({work}, {'logits' if sampler else 'uniform'} sampler, HALF_DARK, after 64 untimed steps)"}


OBS_TIMED_EVERY = 8   # observation launches timed with events: every 8th step of the timed region

# device kernel that writes the observation rows, per output format
OBS_KERNEL = {"f32": "jq::k_observe<0, false>", "bf16": "jq::k_observe<1, false>", "u8": "jq::k_observe_u8_persist"}


def measured_traffic(kernel: str, games: int):
    """HBM bytes per launch of `kernel` (FETCH_SIZE + WRITE_SIZE, scaled against a
    plain copy) from the committed counter summary, when it was taken at this size."""
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None
    rec = json.loads(path.read_text()).get("kernels", {}).get(kernel)
    if not rec or rec.get("games") != games:
        return None
    return round(rec["read_bytes"] + rec["write_bytes"])


def measure(args, path: str) -> dict:
    """Play the batch into mixed stages, then time `args.steps` env-steps of
    `path` (fused / separate / dropin); returns the JSON record without the CPU
    baseline."""
    import numpy as np
    import torch

    import junqi_amd
    from junqi_amd import _lib as L

    cfg = dict(CONFIGS[args.config])
    n = args.envs or cfg["envs"]
    sampler = args.sampler or cfg["sampler"]
    smp = L.SAMPLE_LOGITS if sampler == "logits" else L.SAMPLE_UNIFORM
    stagger = cfg["stagger"] if args.stagger < 0 else args.stagger
    with_obs = cfg["obs"] or path == "dropin"
    fmt = "f32" if path == "dropin" else args.fmt
    b = junqi_amd.JunqiBatch(n, show_mode=args.show_mode, max_num_moves=4000, pool_size=10000)
    b.reset(0)
    b.legal()
    dev = b.device
    es = {"u8": 1, "bf16": 2, "f32": 4}[fmt]
    sdt = {"u8": torch.uint8, "bf16": torch.bfloat16, "f32": torch.float32}[fmt]
    fmt_code = {"u8": L.OBS_U8, "bf16": L.OBS_BF16, "f32": L.OBS_F32}[fmt]
    spatial = torch.empty((n, 317, 17, 17), dtype=sdt, device=dev) if with_obs else None
    aux = torch.empty((n, AUX_BYTES), dtype=torch.uint8, device=dev) if with_obs and fmt == "u8" else None
    glob = torch.empty((n, 28), dtype=torch.float32, device=dev) if with_obs else None
    K = args.steps
    term = torch.empty((K + 1, n), dtype=torch.uint8, device=dev)
    reward = torch.empty((K + 1, n), dtype=torch.float32, device=dev)
    hsh = torch.empty((K + 1, n), dtype=torch.int64, device=dev)
    acts = torch.empty((K + 1, n), dtype=torch.int32, device=dev)
    canon = torch.empty(n, dtype=torch.int32, device=dev)
    mask_bool = torch.empty((n, 16641), dtype=torch.uint8, device=dev) if path == "dropin" else None
    h, lib = b._h, L.lib
    cap = b.values.numel()
    P = lambda t: None if t is None else t.data_ptr()  # noqa: E731

    # ---- mixed stages: game i takes no action during its first S_i steps
    start = torch.from_numpy(np.random.default_rng(7).integers(0, max(1, stagger), n).astype(np.int64)).to(dev)
    for k in range(stagger):
        s = torch.cuda.current_stream(dev).cuda_stream
        a = acts[0]
        if smp == L.SAMPLE_LOGITS:
            L.check(lib.jq_sample_logits(h, None, b.counts.data_ptr(), b.offsets.data_ptr(), b.values.data_ptr(),
                                         cap, args.seed, k, a.data_ptr(), None, s))
        else:
            L.check(lib.jq_sample_uniform(h, b.counts.data_ptr(), b.offsets.data_ptr(), b.values.data_ptr(), cap,
                                          args.seed, k, a.data_ptr(), s))
        a.copy_(torch.where(start > k, torch.full_like(a, -1), a))
        L.check(lib.jq_env_step(h, a.data_ptr(), smp, args.seed, k, k, b.counts.data_ptr(), b.offsets.data_ptr(),
                                b.values.data_ptr(), cap, b.mask_words.data_ptr(), fmt_code, None, None, None,
                                None, None, None, None, s))
    torch.cuda.synchronize(dev)
    plies0 = b.get_field("move_counter")[:, 0]

    def one_step(ply: int, slot: int):
        s = torch.cuda.current_stream(dev).cuda_stream
        if path == "fused":
            # one call: sample from the previous CSR rows, ply, restart, next seat's
            # CSR + mask, observation (the library times the observation kernel)
            L.check(lib.jq_env_step(h, None, smp, args.seed, ply, ply, b.counts.data_ptr(), b.offsets.data_ptr(),
                                    b.values.data_ptr(), cap, b.mask_words.data_ptr(), fmt_code, P(spatial), P(aux),
                                    P(glob), term[slot].data_ptr(), reward[slot].data_ptr(), hsh[slot].data_ptr(),
                                    acts[slot].data_ptr(), s))
            return
        if path == "separate":
            if smp == L.SAMPLE_LOGITS:
                L.check(lib.jq_sample_logits(h, None, b.counts.data_ptr(), b.offsets.data_ptr(),
                                             b.values.data_ptr(), cap, args.seed, ply, acts[slot].data_ptr(), None, s))
            else:
                L.check(lib.jq_sample_uniform(h, b.counts.data_ptr(), b.offsets.data_ptr(), b.values.data_ptr(),
                                              cap, args.seed, ply, acts[slot].data_ptr(), s))
            L.check(lib.jq_step(h, acts[slot].data_ptr(), None, L.ACT_WORLD, None, None, term[slot].data_ptr(),
                                None, None, None, None, reward[slot].data_ptr(), None, s))
            L.check(lib.jq_reset_terminated(h, ply, s))
            L.check(lib.jq_legal(h, None, b.counts.data_ptr(), b.offsets.data_ptr(), b.values.data_ptr(), cap,
                                 b.mask_words.data_ptr(), None, s))
        else:   # GpuRollout's calls: canonical step of the acting seats, device reset, bool mask + CSR
            turn = b.field_tensor("turn").contiguous()   # turn_torch(): the acting seats
            L.check(lib.jq_sample_logits(h, None, b.counts.data_ptr(), b.offsets.data_ptr(), b.values.data_ptr(),
                                         cap, args.seed, ply, acts[slot].data_ptr(), canon.data_ptr(), s))
            L.check(lib.jq_step(h, canon.data_ptr(), turn.data_ptr(), L.ACT_CANONICAL, None, None,
                                term[slot].data_ptr(), None, None, None, None, reward[slot].data_ptr(), None, s))
            L.check(lib.jq_reset_terminated(h, ply, s))
            L.check(lib.jq_legal(h, None, b.counts.data_ptr(), b.offsets.data_ptr(), b.values.data_ptr(), cap,
                                 None, mask_bool.data_ptr(), s))
        if with_obs:
            L.check(lib.jq_observe(h, None, fmt_code, 0, spatial.data_ptr(), P(aux), glob.data_ptr(), s))

    for w in range(args.warmup):
        one_step(stagger + w, K)
    torch.cuda.synchronize(dev)
    t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    total0, n0 = ctypes.c_double(0.0), ctypes.c_int64(0)
    L.check(lib.jq_obs_timing_read(h, ctypes.byref(total0), ctypes.byref(n0)))   # start a new count
    torch.cuda.synchronize(dev)
    wall0 = time.perf_counter()
    t_start.record()
    for k in range(K):
        # HIP events around the observation launch of every OBS_TIMED_EVERY-th step,
        # on its stream (the end event costs that step about 6 us of queue time;
        # the fused call's begin event doubles as the release of its side stream)
        L.check(lib.jq_obs_timing(h, 1 if k % OBS_TIMED_EVERY == 0 else 0))
        one_step(stagger + args.warmup + k, k)
    t_end.record()
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - wall0
    ms_total = t_start.elapsed_time(t_end)
    obs_total, obs_n = ctypes.c_double(0.0), ctypes.c_int64(0)
    L.check(lib.jq_obs_timing_read(h, ctypes.byref(obs_total), ctypes.byref(obs_n)))
    L.check(lib.jq_obs_timing(h, 0))
    obs_ms = obs_total.value / max(1, obs_n.value) if with_obs else None
    kbar = int(b.offsets[-1].item()) / n
    ended = int(term[:K].sum().item())

    steps_per_s = n * K / (ms_total / 1e3)
    obs_bytes = (OBS_ELEMS * es + (AUX_BYTES if fmt == "u8" else 0) + GLOBAL_BYTES) if with_obs else 0
    mask_bytes = 16641 if path == "dropin" else MASK_BYTES
    step_bytes = obs_bytes + mask_bytes + 8 + 4 * kbar + (STEP_OUT_BYTES if path == "fused" else 5)
    whole = step_bytes * steps_per_s / 1e9
    rec = {
        "metric": METRIC,
        "value": round(steps_per_s, 1),
        "unit": "env-steps/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_total / K, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": fmt if with_obs else "int32",
        "data": "synthetic: seeded random legal setups, Philox-sampled legal actions, games played into mixed "
                "stages before timing, auto-reset from a 10000-setup pool",
        "config": {"workload": f"{args.config}: sample ({sampler}) + step + pool restart + sorted legal CSR + "
                               + ("bool canonical mask" if path == "dropin" else "packed canonical mask")
                               + (f" + 317-plane {fmt} obs of the acting seat" if with_obs else "")
                               + f", {n} games, show mode {args.show_mode}",
                   "games": n, "obs_format": fmt if with_obs else None, "path": path, "sampler": sampler,
                   "stagger_steps": stagger, "mean_legal_actions": round(kbar, 2),
                   "plies_at_start": {"min": int(plies0.min()), "mean": round(float(plies0.mean()), 1),
                                      "max": int(plies0.max())},
                   "games_ended_in_window": ended},
        "whole_step": {"bytes_per_env_step": round(step_bytes, 1), "achieved_GBps": round(whole, 1),
                       "frac": round(whole / HBM_PEAK_GBS, 4)},
        "wall_s": round(wall, 3),
    }
    if with_obs:
        per_launch = n * obs_bytes
        achieved = per_launch / (obs_ms / 1e3) / 1e9
        rec["roofline"] = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": round(achieved / HBM_PEAK_GBS, 4),
                           "traffic": measured_traffic(OBS_KERNEL[fmt], n),
                           "kernel": OBS_KERNEL[fmt], "kernel_ms": round(obs_ms, 4), "bytes_per_launch": per_launch}
    else:
        rec["roofline"] = {"bound": "hbm", "achieved": round(whole, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": round(whole / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "whole step",
                           "kernel_ms": round(ms_total / K, 4), "bytes_per_launch": round(step_bytes * n)}
    b.close()
    if with_obs:
        # the same byte count written by a plain device fill: what a write-only
        # kernel can reach on this device, beside the 8 TB/s spec peak
        fill = fill_rate_gbps(per_launch)
        rec["roofline"]["measured_fill_GBps"] = round(fill, 1)
        rec["roofline"]["frac_of_fill"] = round(rec["roofline"]["achieved"] / fill, 4)
    return rec


def main() -> int:
    args = parse()
    if args.calibrate_copy:
        return calibrate_copy(args.calibrate_copy)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the environment shards by games with no exchange "
              "(G GPUs = G independent batches), so it has no multi-GPU run", file=sys.stderr)
        return 2
    import torch

    rec = measure(args, args.path)
    if args.path == "fused" and args.config == "c5" and not args.no_dropin:
        # the same games through the reference collector's unchanged calls: f32
        # observation, bool canonical mask, canonical step, device reset
        torch.cuda.empty_cache()
        d = measure(args, "dropin")
        torch.cuda.empty_cache()
        rec["dropin"] = {"value": d["value"], "unit": d["unit"], "ms_per_step": d["ms_per_step"], "dtype": d["dtype"],
                         "workload": d["config"]["workload"], "steps": d["steps"], "warmup": d["warmup"],
                         "roofline": {k: d["roofline"][k] for k in ("kernel", "kernel_ms", "achieved", "frac")},
                         "whole_step": d["whole_step"]}
    sampler = args.sampler or CONFIGS[args.config]["sampler"]
    with_obs = CONFIGS[args.config]["obs"] or args.path == "dropin"
    if not args.no_cpu:
        rec["cpu_baseline"] = cpu_baseline(args.cpu_envs, args.cpu_seconds, 1 if sampler == "logits" else 0,
                                           with_obs, args.seed)
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
