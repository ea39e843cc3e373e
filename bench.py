#!/usr/bin/env python3
"""Benchmark: one rank's share of exact causal ring attention, forward +
recompute backward, on one MI355X (BASELINE configs 2 and 3).

Workload (one "step"): rank 7 of an 8-rank ring, a 32768-token bf16 local
query shard, Hq = Hkv = 16, d = 128.  Forward: the diagonal KV shard plus 7
preceding full KV shards, each hop's result merged by log-sum-exp into the
running state in the forward kernel's epilogue, then a cast to the bf16
output.  Backward: preprocess
(delta, LSE), then per hop the dK/dV kernel (per-shard dK/dV, as they would
travel back around the ring), which also stores dS (bf16) in a workspace,
and the dQ kernel that reads it back (accumulating dQ across shards);
--bwd-recompute runs the dQ kernel that recomputes S and dP instead.
Inputs (Q, K, V, dO ~ N(0,1), seeded) are resident in HBM before the timed
region; the dS workspace (34 GiB at the default shape) is allocated before
it.

FLOP convention (algorithmic, fully masked tiles not counted): a full
(query shard x KV shard) forward is 4*Nq*Nk*H*d, the diagonal counts half,
the backward is 2.5x the forward.  Peak: bf16 dense MFMA 2516.6 TFLOP/s.

The CPU baseline times the C restatement of the reference algorithm
(oracle/ring_ref.c, OpenMP on the host cores) on a bounded sample: one head
of the same geometry with a shorter shard, sized to ~15 s.

After the headline measurement, with its tensors freed, the default run also
measures the other configurations that fit one GPU in short runs (config 5's
1M-token forward, the C4 prefill attention share, the C4 decode step) and
adds their summaries to the same line under "other_configs";
--no-other-configs skips them.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import socket
import sys
import threading
import time

PEAK_BF16_TFLOPS = 2516.6
PEAK_SCLK_MHZ = 2400.0  # the shader clock the published peak assumes
METRIC = "causal attn fwd+bwd TFLOP/s @32k bf16 shard, % MFMA peak; vs CPU ref"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--tokens", type=int, default=32768, help="local shard tokens")
    ap.add_argument("--world", type=int, default=8)
    ap.add_argument("--rank", type=int, default=7)
    ap.add_argument("--heads", type=int, default=16)
    ap.add_argument("--head-dim", type=int, default=128)
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="target duration of the CPU-baseline sample (0 disables it)")
    ap.add_argument("--c4-prefill", action="store_true",
                    help="time the C4 model's per-layer attention share (GQA 32/8, 65,536 tokens, "
                         "rank 3 of 4, forward) instead of the default workload")
    ap.add_argument("--c4-model", action="store_true",
                    help="time the whole C4 model prefill share (embedding, 24 layers, LM head)")
    ap.add_argument("--c4-decode", action="store_true",
                    help="time incremental decode of the C4 model against a 262,144-token KV cache")
    ap.add_argument("--long-shard", action="store_true",
                    help="BASELINE config 5 instead: forward of a 1,000,000-token bf16 shard "
                         "against its diagonal block plus one full incoming 1M-token KV shard; "
                         "prints its own JSON line with TFLOP/s and the HBM footprint")
    ap.add_argument("--host-path", action="store_true",
                    help="time the host-pointer entry points (lc_ring_*_host: the reference's "
                         "CPU-tensor signatures, PCIe copies included) against the same ring "
                         "entry points on device-resident shards, at configs 2/3")
    ap.add_argument("--bwd-recompute", action="store_true",
                    help="backward without dS sharing: the dQ kernel recomputes S and dP "
                         "instead of reading the dS the dK/dV kernel stored")
    ap.add_argument("--separate-merge", action="store_true",
                    help="forward with each later hop into its own partial buffers and the "
                         "lc_attn_merge kernel per hop, instead of the merge in the forward's "
                         "epilogue (measures the merge kernel's HBM rate in the step)")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the short runs of configs 5, 4 (prefill attention) and the C4 decode "
                         "that follow the headline measurement")
    ap.add_argument("--kernel-power", action="store_true",
                    help="run each ring kernel class of configs 2/3 back to back for ~2 s and "
                         "report its time per launch with the socket power and shader clock "
                         "(amdsmi) it runs at")
    ap.add_argument("--cpu-shard", action="store_true",
                    help="only time the CPU baseline at the workload's own shard size (one head, "
                         "world 2 rank 1: one full hop and the diagonal of --tokens-token shards, "
                         "about 45 s on 16 threads) and print its JSON line; no GPU work")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy (calibrates the "
                         "FETCH_SIZE / WRITE_SIZE counters against known bytes)")
    return ap.parse_args()


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(args, target_s: float):
    """Times the C oracle (the reference's blocked fp32 algorithm) on one head
    of the bench geometry with a shard of n_s tokens, n_s sized so the run
    takes about target_s seconds."""
    import numpy as np

    from oracle import ring as oring

    world, rank, d = args.world, args.rank, args.head_dim

    def run(ns, world=world, rank=rank):
        rng = np.random.default_rng(99)
        mk = lambda: rng.standard_normal((1, ns, 1, d)).astype(np.float32)  # noqa: E731
        qs = [mk() for _ in range(world)]
        ks = [mk() for _ in range(world)]
        vs = [mk() for _ in range(world)]
        go = mk()
        t0 = time.perf_counter()
        out, m, l = oring.ring_fwd_with_stats(qs, ks, vs, rank)
        # other ranks' (out, m, l, dO) only enter pass-1 hops whose pairs are
        # all masked for this rank; any finite values give zero there
        outs = [np.zeros_like(out) for _ in range(world)]
        ms = [np.zeros_like(m) for _ in range(world)]
        ls = [np.ones_like(l) for _ in range(world)]
        gos = [np.zeros_like(go) for _ in range(world)]
        outs[rank], ms[rank], ls[rank], gos[rank] = out, m, l, go
        t1 = time.perf_counter()
        log(f"cpu baseline: {ns}-token shards, world {world} rank {rank}: forward {t1 - t0:.1f} s")
        oring.ring_bwd(qs, ks, vs, outs, ms, ls, gos, rank)
        t2 = time.perf_counter()
        log(f"cpu baseline: backward {t2 - t1:.1f} s")
        return t2 - t0

    if args.cpu_shard:
        # the workload's own shard size on the smallest ring that holds both hop kinds
        ns, world, rank = args.tokens, 2, 1
        t = run(ns, world, rank)
        flops = 3.5 * 4.0 * ns * ns * d * 1.5
        return {
            "value": round(flops / t / 1e12, 6),
            "unit": "TFLOP/s",
            "cores": oring.num_threads(),
            "cpu_model": cpu_model(),
            "kind": "port",
            "sample": (f"C restatement of the reference algorithm (fp32, block_q=64, "
                       f"block_k=128, two-pass backward), 1 head, world 2 rank 1 (one full hop "
                       f"and the diagonal), {ns}-token shards, d={d}: fwd+bwd "
                       f"{flops / 1e9:.1f} GFLOP in {t:.2f} s"),
            "seconds": round(t, 3),
        }

    ns = 256
    t = run(ns)
    while t < target_s / 8 and ns < args.tokens:
        ns = min(args.tokens, ns * 2)
        t = run(ns)
    if t < target_s * 0.6 and ns < args.tokens:
        ns = min(args.tokens, int(ns * math.sqrt(target_s / t)) // 128 * 128)
        t = run(ns)
    hops_full = rank  # owners rank-1 .. 0 are full, owner rank is the diagonal
    fwd = 4.0 * ns * ns * 1 * d * (hops_full + 0.5)
    flops = 3.5 * fwd
    return {
        "value": round(flops / t / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": oring.num_threads(),
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": (f"C restatement of the reference algorithm (fp32, block_q=64, block_k=128, "
                   f"two-pass backward), 1 of {args.heads} heads, world {world} rank {rank}, "
                   f"{ns}-token shards, d={d}: fwd+bwd {flops / 1e9:.1f} GFLOP in {t:.2f} s"),
        "seconds": round(t, 3),
    }


class PowerReader:
    """Socket power (W) and current shader clock (MHz) of the GPU torch runs on,
    through amdsmi's read-only metrics query; ``ok`` is False when amdsmi is
    unavailable or the device cannot be matched by its PCI address."""

    def __init__(self, torch):
        self.ok, self.cap_w = False, None
        try:
            import amdsmi

            amdsmi.amdsmi_init()
            pr = torch.cuda.get_device_properties(0)
            bdf = f"{pr.pci_domain_id:04x}:{pr.pci_bus_id:02x}:{pr.pci_device_id:02x}.0"
            try:
                self.h = amdsmi.amdsmi_get_processor_handle_from_bdf(bdf)
            except Exception:  # noqa: BLE001 - fall back to the only GPU amdsmi sees
                hs = amdsmi.amdsmi_get_processor_handles()
                if len(hs) != 1:
                    return
                self.h = hs[0]
            self.amdsmi = amdsmi
            try:
                cap = amdsmi.amdsmi_get_power_cap_info(self.h).get("power_cap")
                self.cap_w = round(cap / 1e6, 1) if cap else None  # reported in microwatts
            except Exception:  # noqa: BLE001
                pass
            self.ok = self.read() is not None
        except Exception:  # noqa: BLE001 - best effort
            self.ok = False

    def read(self):
        try:
            m = self.amdsmi.amdsmi_get_gpu_metrics_info(self.h)
        except Exception:  # noqa: BLE001
            return None
        w, mhz = m.get("current_socket_power"), m.get("current_gfxclk")
        if not isinstance(w, (int, float)) or w in (0xFFFF, 0xFFFFFFFF):
            return None
        return float(w), (float(mhz) if isinstance(mhz, (int, float)) and mhz != 0xFFFF else None)


class ClockSampler:
    """Samples the GPU's current shader clock (torch.cuda.clock_rate, read
    through amdsmi) every ``period`` seconds while running, so a bench line
    records the clock its kernels ran at: MI355X boxes of one pool differ by
    several percent under these kernels, and every kernel time scales with it.
    Reports None when the clock cannot be read (no amdsmi access)."""

    def __init__(self, torch, period: float = 0.02, power: "PowerReader" = None):
        self.torch, self.period = torch, period
        self.samples = []
        self.power = power if power is not None and power.ok else None
        self.power_samples = []
        self._stop = threading.Event()
        self._thread = None

    def _read(self):
        try:
            return float(self.torch.cuda.clock_rate(0))
        except Exception:  # noqa: BLE001 - best effort: amdsmi may be unavailable
            return None

    def _loop(self):
        while not self._stop.wait(self.period):
            v = self._read()
            if v is None:
                return
            self.samples.append(v)
            if self.power is not None:
                pw = self.power.read()
                if pw is not None:
                    self.power_samples.append(pw[0])

    def __enter__(self):
        if self._read() is not None:
            self._thread = threading.Thread(target=self._loop, daemon=True)
            self._thread.start()
        return self

    def __exit__(self, *exc):
        self._stop.set()
        if self._thread is not None:
            self._thread.join()

    # Readings below this are not the clock of a GPU busy with these kernels (under
    # rocprofv3 most readings come back at the 158 MHz idle level): they are dropped,
    # and with fewer than half the readings left there is no summary.
    MIN_BUSY_MHZ = 500.0

    def power_summary(self):
        """Socket power while the timed region ran (W), and the board's cap."""
        xs = self.power_samples
        if not xs:
            return None
        return {"mean": round(sum(xs) / len(xs), 1), "max": max(xs), "samples": len(xs),
                "cap": self.power.cap_w}

    def summary(self):
        xs = [x for x in self.samples if x >= self.MIN_BUSY_MHZ]
        if not xs or 2 * len(xs) < len(self.samples):
            return None
        return {"mean": round(sum(xs) / len(xs), 1), "median": sorted(xs)[len(xs) // 2],
                "min": min(xs), "max": max(xs), "samples": len(xs),
                "dropped_below_500": len(self.samples) - len(xs)}


def measured_traffic(rl_kernel: str, n: int, h: int, d: int):
    """HBM bytes per launch of the roofline kernel(s), from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (calibrated against a plain
    copy); None when the workload is not the one that summary measured."""
    if (n, h, d) != (32768, 16, 128):
        return None
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "hbm_traffic_ring_fwd_bwd_32k_bf16.md")
    try:
        text = open(path).read()
        block = text.split("```json", 1)[1].split("```", 1)[0]
        per = json.loads(block)["traffic_bytes_per_full_hop"]
    except (OSError, IndexError, KeyError, ValueError):
        return None
    names = [part.split()[0] for part in rl_kernel.split(" + ")]
    if not all(k in per for k in names):
        return None  # a kernel of this roofline has no committed traffic measurement
    return sum(per[k] for k in names)


def algorithmic_bytes(rl_kernel: str, n: int, h: int, d: int) -> int:
    """HBM bytes the mathematics of one full hop has to move, for the roofline
    kernel(s): the backward pair reads Q, dO, K, V (bf16) and the two row
    statistics (LSE, delta; fp32) and read-modify-writes dQ, dK, dV (fp32);
    the merging forward reads Q, K, V and read-modify-writes the running fp32
    output and its (m, l).  The dS the dK/dV kernel stores and the dQ kernel
    reads back (bf16, N x N x H) is a choice of this design, not part of the
    floor."""
    bf16_in, f32_row, f32_stat = n * h * d * 2, n * h * d * 4, n * h * 4
    if rl_kernel.startswith("dkdv128_kernel + dqds128_kernel") or \
            rl_kernel.startswith("dq128_kernel + dkdv128_kernel"):
        return 4 * bf16_in + 2 * f32_stat + 3 * 2 * f32_row
    if rl_kernel.startswith("fwd128_kernel"):
        return 3 * bf16_in + 2 * f32_row + 2 * 2 * f32_stat
    return 0


def long_shard_line(torch, ra, steps: int, warmup: int) -> dict:
    """rank 1 of a 2-shard layout with 1,000,000 local tokens,
    Hq = Hkv = 16, d = 128, bf16; forward over the diagonal block and one full
    incoming shard, merged by LSE (1M mod 128 = 64, so every kernel runs tail tiles)."""
    n, h, d = 1_000_000, 16, 128
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(4321)
    bf = torch.bfloat16
    torch.cuda.reset_peak_memory_stats()
    randn = lambda *s: torch.randn(*s, generator=gen, device=dev, dtype=torch.float32).to(bf)  # noqa: E731
    log(f"long shard: n={n} H={h} d={d} bf16, diagonal + 1 full shard")
    q = randn(1, n, h, d)
    k = [randn(1, n, h, d) for _ in range(2)]
    v = [randn(1, n, h, d) for _ in range(2)]
    from longctx100m_amd.rank_step import LongShardForward

    lsf = LongShardForward(q, k, v)

    def step():
        lsf.forward()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    log("long shard: warmup done")
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        step()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    flops = 1.5 * 4.0 * n * n * h * d
    resident = sum(x.numel() * x.element_size() for x in lsf.resident())
    line = {
        "metric": "causal attn fwd TFLOP/s @1M-token bf16 shard (diagonal + 1 full shard)",
        "value": round(flops / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": steps, "ms_per_step": round(ms, 2), "higher_is_better": True,
        "pct_mfma_peak": round(100.0 * flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
        "dtype": "bf16", "data": "synthetic: Q, K, V ~ N(0,1), seeded",
        "config": {"workload": "BASELINE config 5: 1,000,000 local tokens, Hq=Hkv=16, d=128, "
                               "diagonal + 1 full incoming 1M-token KV shard, LSE merge",
                   "local_tokens": n, "heads_q": h, "heads_kv": h, "head_dim": d},
        "flops_per_step": flops,
        "hbm_footprint_gb": {"resident_tensors": round(resident / 1e9, 3),
                             "torch_peak_allocated": round(torch.cuda.max_memory_allocated() / 1e9, 3)},
    }
    return line


def long_shard(args, torch, ra) -> int:
    line = long_shard_line(torch, ra, max(1, min(args.steps, 2)), max(0, min(args.warmup, 1)))
    print(json.dumps(line), flush=True)
    return 0


def kernel_power(args, torch, ra) -> int:
    """Socket power and shader clock under each kernel class of one full hop at
    configs 2/3 (rank 7 of 8: queries at 7 n, keys at 0; bf16, 16 heads, d = 128),
    each launched back to back for ~2 s: the merging forward; the benched
    backward pair (dK/dV storing dS, then dQ from dS); the dK/dV kernel alone
    without dS stores; the recomputing dQ kernel."""
    n, h, d = args.tokens, args.heads, args.head_dim
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(4242)
    bf = torch.bfloat16
    randn = lambda *sh: torch.randn(*sh, generator=gen, device=dev).to(bf)  # noqa: E731
    q, k, v, do = (randn(1, n, h, d) for _ in range(4))
    qp = 7 * n
    o, m, l = ra.fwd_shard(q, k, v, q_pos0=qp, k_pos0=0)
    out = torch.empty_like(q)
    ra.cast(o, out)
    delta, lse2 = ra.bwd_preprocess(out, do, m, l)
    f32 = dict(device=dev, dtype=torch.float32)
    dq, dk, dv = (torch.zeros(1, n, h, d, **f32) for _ in range(3))
    ws = torch.empty(ra.bwd_shard_workspace_bytes(q, k), dtype=torch.uint8, device=dev)
    args_b = (q, k, v, do, lse2, delta)
    unit = 4.0 * n * n * h * d
    kernels = {
        "fwd128_kernel<8> (merging full hop)": (unit, lambda: ra.fwd_shard(
            q, k, v, q_pos0=qp, k_pos0=0, o=o, m=m, l=l, accumulate=True)),
        "dkdv128_kernel + dqds128_kernel (the benched pair)": (2.5 * unit, lambda: ra.bwd_shard(
            *args_b, q_pos0=qp, k_pos0=0, dq_acc=dq, dk_acc=dk, dv_acc=dv, workspace=ws)),
        "dkdv128_kernel without dS stores": (2.0 * unit, lambda: ra.bwd_shard(
            *args_b, q_pos0=qp, k_pos0=0, dk_acc=dk, dv_acc=dv)),
        "dq128_kernel (recomputing S and dP)": (1.5 * unit, lambda: ra.bwd_shard(
            *args_b, q_pos0=qp, k_pos0=0, dq_acc=dq)),
    }
    pr = PowerReader(torch)
    res = {}
    for name, (flops, fn) in kernels.items():
        fn()
        torch.cuda.synchronize()
        reps, t0 = 0, time.perf_counter()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with ClockSampler(torch, period=0.05, power=pr) as clock:
            a.record()
            while time.perf_counter() - t0 < 2.0:
                for _ in range(4):
                    fn()
                    reps += 1
                torch.cuda.synchronize()
            b.record()
            b.synchronize()
        ms = a.elapsed_time(b) / reps
        res[name] = {"ms_per_launch": round(ms, 3), "launches": reps,
                     "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
                     "power_w": clock.power_summary(), "sclk_mhz": clock.summary()}
        log(f"{name}: {ms:.3f} ms, power {res[name]['power_w']}, clock {res[name]['sclk_mhz']}")
    print(json.dumps({"metric": "socket power and shader clock per ring kernel class (one full "
                                "hop, configs 2/3)", "power_cap_w": pr.cap_w if pr.ok else None,
                      "kernels": res, "box": socket.gethostname()}), flush=True)
    return 0


def host_path_line(torch, ra, steps: int, warmup: int, n: int = 32768, h: int = 16,
                   d: int = 128, world: int = 8, rank: int = 7) -> dict:
    """The reference's signatures (ring_causal_attention_forward_with_stats,
    ring_causal_attention_backward: rs:139-233, rs:281-475) at configs 2/3
    shapes: on shards already in HBM (lc_ring_fwd_with_stats, then lc_ring_bwd
    with the workspace of lc_ring_bwd_ds_workspace_bytes, which shares dS on
    the diagonal pair), and on host memory (lc_ring_fwd_with_stats_host,
    lc_ring_bwd_host: every call copies all ranks' shards to HBM and the
    results back).  Both run the same kernels; the difference is the PCIe
    traffic.  value = device-resident forward + backward, ms per call."""
    import ctypes

    import numpy as np

    from longctx100m_amd import _lib

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(97)
    bf = torch.bfloat16
    randn = lambda *sh: torch.randn(*sh, generator=gen, device=dev).to(bf)  # noqa: E731
    log(f"host path: world={world} rank={rank} n={n} H={h} d={d} bf16")
    qs = [randn(1, n, h, d) for _ in range(world)]
    ks = [randn(1, n, h, d) for _ in range(world)]
    vs = [randn(1, n, h, d) for _ in range(world)]
    gos = [randn(1, n, h, d) for _ in range(world)]
    shards = list(zip(qs, ks, vs))
    out, m, l = ra.ring_causal_attention_forward_with_stats(shards, rank)
    outs, ms, ls = [out] * world, [m] * world, [l] * world
    torch.cuda.synchronize()
    host = lambda t: np.ascontiguousarray(t.cpu().view(torch.int16).numpy())  # noqa: E731
    hq, hk, hv, hg = ([host(t) for t in ts] for ts in (qs, ks, vs, gos))
    ho, hm, hl = host(out), np.ascontiguousarray(m.cpu().numpy()), np.ascontiguousarray(l.cpu().numpy())
    desc = _lib.RingDesc(world, rank, 1, n, h, h, d, _lib.LC_DTYPE_BF16, 0, 1, 64, 128, -1, -1)
    lib = _lib.load()
    ptrs = lambda arrs: _lib.ptr_array([a.ctypes.data for a in arrs])  # noqa: E731
    P = [ptrs(x) for x in (hq, hk, hv, [ho] * world, [hm] * world, [hl] * world, hg)]
    o_h = np.empty_like(ho)
    m_h, l_h = np.empty_like(hm), np.empty_like(hl)
    dq_h, dk_h, dv_h = np.empty_like(ho), np.empty_like(ho), np.empty_like(ho)

    def fwd_host():
        _lib.check(lib.lc_ring_fwd_with_stats_host(ctypes.byref(desc), P[0][0], P[1][0], P[2][0],
                                                   o_h.ctypes.data, m_h.ctypes.data,
                                                   l_h.ctypes.data))

    def bwd_host():
        _lib.check(lib.lc_ring_bwd_host(ctypes.byref(desc), *[x[0] for x in P], dq_h.ctypes.data,
                                        dk_h.ctypes.data, dv_h.ctypes.data))

    def fwd_dev():
        ra.ring_causal_attention_forward_with_stats(shards, rank)

    def bwd_dev():
        ra.ring_causal_attention_backward(shards, rank, outs, ms, ls, gos)

    def wall(fn, reps):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / reps

    reps = max(1, steps)
    res = {"fwd_host_s": wall(fwd_host, reps), "fwd_device_s": wall(fwd_dev, reps),
           "bwd_host_s": wall(bwd_host, reps), "bwd_device_s": wall(bwd_dev, reps)}
    shard = n * h * d * 2
    stat = h * n * 4
    fwd_bytes = (1 + 2 * world) * shard + shard + 2 * stat      # Q + all K, V in; out, m, l back
    bwd_bytes = world * (5 * shard + 2 * stat) + 3 * shard      # q, k, v, out, dO, m, l per rank in; dq, dk, dv back
    line = {
        "metric": "reference-signature ring fwd+bwd (lc_ring_fwd_with_stats + lc_ring_bwd), "
                  "device-resident ms per call; host-pointer (PCIe-inclusive) seconds alongside",
        "value": round(1e3 * (res["fwd_device_s"] + res["bwd_device_s"]), 2),
        "unit": "ms", "steps": reps, "ms_per_step": round(1e3 * (res["fwd_device_s"] + res["bwd_device_s"]), 2),
        "n_gpus": 1, "higher_is_better": False, "dtype": "bf16",
        "data": "synthetic: Q, K, V, dO ~ N(0,1), seeded; host copies in pageable memory",
        "config": {"workload": f"BASELINE configs 2/3 shapes through the reference signatures: "
                               f"rank {rank} of {world}, {n}-token shards, Hq=Hkv={h}, d={d}",
                   "note": "ring_causal_attention_backward returns this rank's dq, dk, dv "
                           "(rs:281-475): dQ over all 8 hops, dK/dV of its own shard"},
        **{k: round(v, 4) for k, v in res.items()},
        "bytes_copied": {"fwd": fwd_bytes, "bwd": bwd_bytes},
        "effective_copy_GB_per_s": {
            "fwd": round(fwd_bytes / max(res["fwd_host_s"] - res["fwd_device_s"], 1e-9) / 1e9, 1),
            "bwd": round(bwd_bytes / max(res["bwd_host_s"] - res["bwd_device_s"], 1e-9) / 1e9, 1)},
        "bwd_ds_workspace_bytes": int(lib.lc_ring_bwd_ds_workspace_bytes(ctypes.byref(desc))),
    }
    return line


def host_path(args, torch, ra) -> int:
    line = host_path_line(torch, ra, max(1, min(args.steps, 3)), 1, args.tokens, args.heads,
                          args.head_dim, args.world, args.rank)
    print(json.dumps(line), flush=True)
    return 0


def c4_prefill_line(torch, ra, steps: int, warmup: int) -> dict:
    """The C4 model's attention share on one GPU (prefill): GQA Hq=32 / Hkv=8,
    d=128, bf16, 65,536 local tokens at rank 3 of a 4-rank ring, i.e. the
    diagonal block plus 3 preceding 65,536-token KV shards, merged by LSE.
    One step is one layer's attention; the model has 24 such layers."""
    n, hq, hkv, d, world, rank = 65536, 32, 8, 128, 4, 3
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(2468)
    bf = torch.bfloat16
    torch.cuda.reset_peak_memory_stats()
    randn = lambda *s: torch.randn(*s, generator=gen, device=dev, dtype=torch.float32).to(bf)  # noqa: E731
    log(f"C4 prefill attention: n={n} Hq={hq} Hkv={hkv} d={d} bf16, rank {rank} of {world}")
    shards = [(randn(1, n, hq, d), randn(1, n, hkv, d), randn(1, n, hkv, d)) for _ in range(world)]

    def step():
        return ra.ring_causal_attention_forward_with_stats(shards, rank)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    log("C4 prefill attention: warmup done")
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        step()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    flops = (rank + 0.5) * 4.0 * n * n * hq * d
    line = {
        "metric": "C4 prefill attention TFLOP/s per layer (one GPU's share, GQA 32/8)",
        "value": round(flops / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": steps, "ms_per_step": round(ms, 2), "higher_is_better": True,
        "pct_mfma_peak": round(100.0 * flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
        "dtype": "bf16", "data": "synthetic: Q, K, V ~ N(0,1), seeded",
        "config": {"workload": "C4 model attention share: 65,536 local tokens at rank 3 of 4, "
                               "diagonal + 3 preceding KV shards, LSE merge; one layer",
                   "local_tokens": n, "heads_q": hq, "heads_kv": hkv, "head_dim": d,
                   "layers_in_model": 24},
        "flops_per_step": flops,
        "model_attention_ms_24_layers": round(24 * ms, 1),
        "hbm_peak_allocated_gb": round(torch.cuda.max_memory_allocated() / 1e9, 3),
    }
    return line


def c4_prefill(args, torch, ra) -> int:
    line = c4_prefill_line(torch, ra, max(1, min(args.steps, 3)), max(0, min(args.warmup, 1)))
    print(json.dumps(line), flush=True)
    return 0


def c4_model_line(torch, ra, steps: int, warmup: int) -> dict:
    """the C4 model's prefill on one GPU's share.  Token ids
    of a 65,536-token local shard -> embedding -> 24 decoder layers (RMSNorm,
    fused QKV GEMM, RoPE, ring attention at rank 3 of 4 over the diagonal block
    and 3 preceding KV shards, O GEMM, RMSNorm, fused gate/up GEMM, SwiGLU,
    down GEMM; residual adds fused into the norms) -> final RMSNorm -> LM head.
    Random-init bf16 weights N(0, 0.02); the preceding ranks' K/V shards are
    seeded random tensors per layer."""
    from longctx100m_amd import layer as ly

    cfg = ly.C4
    n, rank, world, d = 65536, 3, 4, cfg.head_dim
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1357)
    bf = torch.bfloat16
    torch.cuda.reset_peak_memory_stats()
    log(f"C4 model prefill: {cfg.num_layers} layers, hidden {cfg.hidden_size}, "
        f"GQA {cfg.num_heads}/{cfg.num_key_value_heads}, {n} tokens at rank {rank} of {world}")
    randn = lambda *s: (torch.randn(*s, generator=gen, device=dev, dtype=torch.float32) * 0.02).to(bf)  # noqa: E731
    embed = randn(cfg.vocab_size, cfg.hidden_size)
    lm_head = randn(cfg.vocab_size, cfg.hidden_size)
    final_norm = torch.ones(cfg.hidden_size, device=dev, dtype=bf)
    layers = [ly.init_layer_weights(cfg, gen, dev) for _ in range(cfg.num_layers)]
    kv = [[(torch.randn(1, n, cfg.num_key_value_heads, d, generator=gen, device=dev).to(bf),
            torch.randn(1, n, cfg.num_key_value_heads, d, generator=gen, device=dev).to(bf))
           for _ in range(rank)] for _ in range(cfg.num_layers)]
    ids = torch.randint(0, cfg.vocab_size, (n,), generator=gen, device=dev)
    table = ly.rope_table(ly.rope_params(d, cfg.rope_theta, cfg.rope_scaling), n, rank * n)
    log("C4 model prefill: weights and inputs ready")

    def prefill(timers=None):
        x = torch.nn.functional.embedding(ids, embed)
        res = None
        for li in range(cfg.num_layers):
            x, res = ly.layer_prefill(x, layers[li], cfg, table, rank, kv[li], residual=res,
                                      timers=timers if li == 0 else None)
        h = ly.rmsnorm(x, final_norm, cfg.rms_norm_eps, residual=res)
        return torch.matmul(h, lm_head.t())

    for _ in range(warmup):
        prefill()
    torch.cuda.synchronize()
    log("C4 model prefill: warmup done")
    timers = {}
    steps = max(1, steps)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        logits = prefill(timers)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    # per-category time of the first layer (last timed step)
    ev = timers.get("_events", [])[-13:]
    cat = {}
    for (_, a), (name, b) in zip(ev, ev[1:]):
        cat[name] = cat.get(name, 0.0) + a.elapsed_time(b)
    fl = ly.layer_flops(cfg, n, rank)
    head = 2.0 * n * cfg.hidden_size * cfg.vocab_size
    flops = cfg.num_layers * (fl["gemm"] + fl["attention"]) + head
    line = {
        "metric": "C4 model prefill TFLOP/s (one GPU's share: 65,536 tokens at rank 3 of 4)",
        "value": round(flops / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": steps, "ms_per_step": round(ms, 1), "higher_is_better": True,
        "pct_mfma_peak": round(100.0 * flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
        "tokens_per_s": round(n / (ms * 1e-3), 1),
        "dtype": "bf16",
        "data": "synthetic: token ids uniform over the vocab, weights N(0,0.02), preceding KV "
                "shards N(0,1), seeded",
        "config": {"workload": "BASELINE config 4: 24-layer Llama-style prefill share, hidden 4096, "
                               "Hq=32, Hkv=8, d=128, SwiGLU 14336, vocab 128256, 65,536 local "
                               "tokens + 3 preceding KV shards per layer",
                   "local_tokens": n, "layers": cfg.num_layers},
        "flops_per_step": flops,
        "flops_split": {"attention": cfg.num_layers * fl["attention"],
                        "gemm": cfg.num_layers * fl["gemm"] + head},
        "layer0_ms": {k: round(v, 3) for k, v in cat.items()},
        "logits_shape": list(logits.shape),
        "hbm_peak_allocated_gb": round(torch.cuda.max_memory_allocated() / 1e9, 2),
    }
    return line


def c4_model(args, torch, ra) -> int:
    line = c4_model_line(torch, ra, max(1, min(args.steps, 2)), max(0, min(args.warmup, 1)))
    print(json.dumps(line), flush=True)
    return 0


def c4_decode_line(torch, ra, steps: int, warmup: int) -> dict:
    """Incremental decode of the C4 model on one GPU: one new token against a
    KV cache of 262,144 tokens per layer (the 4 x 65,536-token context of
    config 4), through embedding, 24 layers (GEMVs, RoPE, split-KV decode
    attention over the cache, SwiGLU) and the LM head.  The reference
    recomputes the full prefill for every generated token
    (distributed_infer.py:185-219, bin/infer.rs:96-106); this is the KV-cache
    step that replaces it.  Cache contents and weights are seeded random."""
    from longctx100m_amd import layer as ly

    cfg = ly.C4
    ctx, d, hkv = 4 * 65536, cfg.head_dim, cfg.num_key_value_heads
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(97531)
    torch.cuda.reset_peak_memory_stats()
    log(f"C4 decode: {cfg.num_layers} layers, KV cache of {ctx} tokens per layer")
    weights = ly.init_model_weights(cfg, gen, dev)
    cap = ctx + steps + warmup + 1
    caches = []
    for _ in range(cfg.num_layers):
        caches.append(tuple(torch.randn(1, cap, hkv, d, generator=gen, device=dev).to(torch.bfloat16)
                            for _ in range(2)))
    table = ly.rope_table(ly.rope_params(d, cfg.rope_theta, cfg.rope_scaling), cap, 0)
    q = torch.zeros(1, 1, cfg.num_heads, d, device=dev, dtype=torch.bfloat16)
    sh = ra._shape(q, caches[0][0], False)
    import ctypes as _ct
    ws = torch.empty(max(1, ra._lib.load().lc_attn_decode_workspace_bytes(_ct.byref(sh))),
                     dtype=torch.uint8, device=dev)
    log("C4 decode: weights and caches ready")
    pos = ctx
    for _ in range(warmup):
        ly.model_decode_step(7, pos, weights, cfg, table, caches, ws)
        pos += 1
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(steps):
        logits = ly.model_decode_step(11 + i, pos, weights, cfg, table, caches, ws)
        pos += 1
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    # the decode attention of one layer alone, at the same context
    qx = torch.randn(1, 1, cfg.num_heads, d, generator=gen, device=dev).to(torch.bfloat16)
    kc, vc = caches[0][0][:, :pos], caches[0][1][:, :pos]
    ra.decode(qx, kc, vc, q_pos0=pos - 1, workspace=ws)
    a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 20
    a0.record()
    for _ in range(reps):
        ra.decode(qx, kc, vc, q_pos0=pos - 1, workspace=ws)
    a1.record()
    torch.cuda.synchronize()
    att_ms = a0.elapsed_time(a1) / reps
    att_bytes = 2.0 * pos * hkv * d * 2
    wbytes = sum(t.numel() * t.element_size() for lw in weights["layers"] for t in lw.values()) + \
        weights["lm_head"].numel() * 2 + cfg.hidden_size * 2
    cache_bytes = cfg.num_layers * att_bytes
    line = {
        "metric": "C4 decode ms per token (one GPU, 262,144-token KV cache per layer)",
        "value": round(ms, 3), "unit": "ms/token", "n_gpus": 1, "steps": steps,
        "ms_per_step": round(ms, 3), "higher_is_better": False,
        "tokens_per_s": round(1e3 / ms, 1),
        "dtype": "bf16", "data": "synthetic: seeded random weights N(0,0.02) and KV cache N(0,1)",
        "config": {"workload": "config 4 model, incremental decode of one token at context "
                               "262,144 (24 layers, GQA 32/8, d=128)", "context": ctx,
                   "layers": cfg.num_layers},
        "hbm_bytes_per_token": {"kv_cache": cache_bytes, "weights": wbytes},
        "roofline": {"bound": "hbm", "achieved": round((cache_bytes + wbytes) / (ms * 1e-3) / 1e9, 1),
                     "peak": 8000.0, "unit": "GB/s",
                     "frac": round((cache_bytes + wbytes) / (ms * 1e-3) / 8e12, 4),
                     "traffic": None, "kernel": "whole decode step (cache + weight reads)"},
        "decode_attention_one_layer": {"ms": round(att_ms, 4), "bytes": att_bytes,
                                       "GB_per_s": round(att_bytes / (att_ms * 1e-3) / 1e9, 1)},
        "vs_prefill_recompute_ms": "the reference's loop reruns the 65,536-token prefill share per token "
                                   "(bench.py --c4-model)",
        "logits_shape": list(logits.shape),
        "hbm_peak_allocated_gb": round(torch.cuda.max_memory_allocated() / 1e9, 2),
    }
    return line


def c4_decode(args, torch, ra) -> int:
    line = c4_decode_line(torch, ra, max(1, args.steps), max(0, args.warmup))
    print(json.dumps(line), flush=True)
    return 0


# Measured after the headline line's timed region (and its CPU baseline) with
# its tensors freed: name -> (measuring function, timed steps, warmup steps).
OTHER_CONFIGS = {
    "c5_long_shard_fwd": (long_shard_line, 1, 1),
    "c4_prefill_attention": (c4_prefill_line, 2, 1),
    "c4_model_prefill": (c4_model_line, 1, 1),
    "c4_decode": (c4_decode_line, 5, 2),
    "reference_signature_c2": (host_path_line, 2, 1),
}
SUMMARY_KEYS = ("metric", "value", "unit", "higher_is_better", "steps", "ms_per_step", "tokens_per_s",
                "fwd_device_s", "bwd_device_s", "fwd_host_s", "bwd_host_s",
                "pct_mfma_peak", "roofline", "config")


def other_configs(torch, ra) -> dict:
    """The other BASELINE configurations that fit one GPU, each a short run:
    the summary of the line its own flag prints (the full line comes from
    bench.py --long-shard / --c4-prefill / --c4-model / --c4-decode /
    --host-path)."""
    out = {}
    for name, (fn, steps, warmup) in OTHER_CONFIGS.items():
        t0 = time.perf_counter()
        try:
            line = fn(torch, ra, steps, warmup)
        except (RuntimeError, ValueError) as e:  # e.g. out of memory: the headline still prints
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
            out[name] = {"error": f"{type(e).__name__}: {e}"[:300]}
            log(f"{name}: failed ({out[name]['error']})")
            continue
        torch.cuda.empty_cache()
        out[name] = {k: line[k] for k in SUMMARY_KEYS if k in line}
        out[name]["wall_s"] = round(time.perf_counter() - t0, 1)
        log(f"{name}: {line['value']} {line['unit']} ({out[name]['wall_s']} s)")
    return out


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU's share of the ring; --gpus {args.gpus} is not "
              f"supported (this build runs on one GPU only)", file=sys.stderr)
        return 2

    import torch

    if args.copy_calibration:
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda:0")  # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copy calibration: 3 copies of 1 GiB (1048576 KiB read + written each)")
        return 0

    if args.cpu_shard:
        cpu = cpu_baseline(args, 0.0)
        # configs 2+3 count 7.5 full hops of forward per head, 3.5x that with the backward
        full = 3.5 * 4.0 * args.tokens ** 2 * args.head_dim * (args.rank + 0.5) * args.heads
        cpu["extrapolated_full_config_s"] = round(full / (cpu["value"] * 1e12), 1)
        print(json.dumps({"metric": "cpu baseline at the workload's shard size",
                          "cpu_baseline": cpu}), flush=True)
        return 0

    from longctx100m_amd import ring_attention as ra

    if args.long_shard:
        return long_shard(args, torch, ra)
    if args.host_path:
        return host_path(args, torch, ra)
    if args.kernel_power:
        return kernel_power(args, torch, ra)
    if args.c4_prefill:
        return c4_prefill(args, torch, ra)
    if args.c4_model:
        return c4_model(args, torch, ra)
    if args.c4_decode:
        return c4_decode(args, torch, ra)

    from longctx100m_amd.rank_step import RankStep

    torch.cuda.set_device(0)
    dev = torch.device("cuda:0")
    n, h, d, world, rank = args.tokens, args.heads, args.head_dim, args.world, args.rank
    bf = torch.bfloat16
    log(f"setup: world={world} rank={rank} n={n} H={h} d={d} bf16")
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    randn = lambda *s: torch.randn(*s, generator=gen, device=dev, dtype=torch.float32).to(bf)  # noqa: E731
    q = randn(1, n, h, d)
    dout = randn(1, n, h, d)
    ks = [randn(1, n, h, d) for _ in range(world)]
    vs = [randn(1, n, h, d) for _ in range(world)]
    rs = RankStep(q, dout, ks, vs, rank, share_ds=not args.bwd_recompute,
                  separate_merge=args.separate_merge)
    owners = rs.owners
    ws = rs.workspace
    shares_ds = ws is not None
    if ws is not None:
        log(f"dS exchange workspace: {ws.numel() / 2**30:.1f} GiB")

    timers = {}

    def timed(name, fn):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        timers.setdefault(name, []).append((s, e))

    def step(record: bool):
        rs.step(timed if record else None)

    for i in range(args.warmup):
        step(False)
        torch.cuda.synchronize()
        log(f"warmup step {i + 1}/{args.warmup} done")

    torch.cuda.synchronize()
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    with ClockSampler(torch, power=PowerReader(torch)) as clock:
        t_start.record()
        for i in range(args.steps):
            step(True)
        t_end.record()
        torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_total = t_start.elapsed_time(t_end)
    ms_per_step = ms_total / args.steps
    log(f"timed {args.steps} steps: {ms_per_step:.3f} ms/step (wall {wall:.2f} s)")

    kern = {}
    for name, evs in timers.items():
        durs = [s.elapsed_time(e) for s, e in evs]
        kern[name] = {"launches_per_step": len(durs) // args.steps,
                      "avg_ms": round(sum(durs) / len(durs), 4)}

    n_full = sum(1 for b in owners if b != rank)
    has_diag = rank in owners
    unit = 4.0 * n * n * h * d  # forward flops of one full (Q shard x KV shard) pair
    fwd_flops = unit * (n_full + (0.5 if has_diag else 0.0))
    total_flops = 3.5 * fwd_flops
    tflops = total_flops / (ms_per_step * 1e-3) / 1e12

    # Dominant kernel class by time per step; roofline against the bf16 MFMA peak.
    tot = {k: v["avg_ms"] * v["launches_per_step"] for k, v in kern.items()}
    fwd_t = tot.get("fwd_full", 0.0) + tot.get("fwd_diag", 0.0)
    bwd_t = sum(tot.get(k, 0.0) for k in ("dq_full", "dq_diag", "dkdv_full", "dkdv_diag",
                                          "bwd_full", "bwd_diag"))
    if n_full > 0 and bwd_t >= fwd_t:
        if "bwd_full" in kern:
            pair_ms = kern["bwd_full"]["avg_ms"]
            rl_kernel = "dkdv128_kernel + dqds128_kernel (one full hop)"
        else:
            pair_ms = kern["dq_full"]["avg_ms"] + kern["dkdv_full"]["avg_ms"]
            rl_kernel = "dq128_kernel + dkdv128_kernel (one full hop)"
        achieved = 2.5 * unit / (pair_ms * 1e-3) / 1e12
        rl_units = f"2.5 x 4*N*N*H*d = {2.5 * unit / 1e12:.3f} TFLOP per full hop"
    elif n_full > 0:
        achieved = unit / (kern["fwd_full"]["avg_ms"] * 1e-3) / 1e12
        rl_kernel = "fwd128_kernel (one full hop)"
        rl_units = f"4*N*N*H*d = {unit / 1e12:.3f} TFLOP per full hop"
    else:
        achieved = tflops
        rl_kernel = "whole step"
        rl_units = f"{total_flops / 1e12:.3f} TFLOP per step"
    sclk = clock.summary()
    traffic = measured_traffic(rl_kernel, n, h, d)
    alg_bytes = algorithmic_bytes(rl_kernel, n, h, d)
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                "traffic": traffic, "kernel": rl_kernel,
                "algorithmic": rl_units,
                # HBM bytes the mathematics of the hop needs (no dS exchange), and how many
                # times that the kernels move (the dS round trip is most of the excess)
                "traffic_algorithmic": alg_bytes or None,
                "traffic_over_algorithmic": (round(traffic / alg_bytes, 2)
                                             if traffic and alg_bytes else None),
                "ds_exchange_bytes": (2 * n * n * h * 2 if "dqds128" in rl_kernel else 0),
                "sclk_mhz": sclk,
                # socket power over the timed region (amdsmi), against the board's cap
                "power_w": clock.power_summary(),
                # the same fraction against the peak scaled to the mean sampled shader clock
                # (the 2516.6 TFLOP/s peak assumes 2.4 GHz; the samples are the firmware's
                # clock levels, so this is approximate): comparable across boxes
                "frac_at_sampled_clock": (
                    round(achieved / (PEAK_BF16_TFLOPS * sclk["mean"] / PEAK_SCLK_MHZ), 4)
                    if sclk and sclk["mean"] > 0 else None),
                "box": socket.gethostname()}

    del rs, q, dout, ks, vs, ws
    torch.cuda.empty_cache()
    others = None if args.no_other_configs else other_configs(torch, ra)

    cpu = None
    if args.cpu_seconds > 0:
        log("cpu baseline (C restatement of the reference algorithm) ...")
        cpu = cpu_baseline(args, args.cpu_seconds)
        # the same restatement on the whole workload of this line, at the sample's rate
        cpu["extrapolated_full_config_s"] = round(total_flops / (cpu["value"] * 1e12), 1)
        log(f"cpu baseline: {cpu['value']} TFLOP/s on {cpu['cores']} threads ({cpu['seconds']} s) "
            f"of {cpu['cpu_model']}; full config extrapolated: "
            f"{cpu['extrapolated_full_config_s']} s")

    line = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: Q, K, V, dO ~ N(0,1) (seeded torch generator), resident in HBM",
        "config": {
            "workload": (f"BASELINE configs 2+3: rank {rank} of {world}, {n}-token bf16 local "
                         f"shard, Hq=Hkv={h}, d={d}; fwd over diagonal + {n_full} full KV shards "
                         f"with LSE merge" + (" (merge kernel per hop)" if args.separate_merge
                                              else "") + ", then recompute bwd (dQ across shards, dK/dV per "
                         f"shard; " + ("dS shared by the dK/dV and dQ kernels)" if shares_ds
                                       else "dQ kernel recomputes dS)")),
            "world": world, "rank": rank, "local_tokens": n, "heads_q": h, "heads_kv": h,
            "head_dim": d, "parallelism": "one rank's share on one GPU (ring emulated in HBM)",
        },
        "pct_mfma_peak": round(100.0 * tflops / PEAK_BF16_TFLOPS, 2),
        "flops_per_step": total_flops,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": kern,
        "other_configs": others,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
