#!/usr/bin/env python3
"""PPO minibatch step throughput on one MI355X.

One step = one PPO minibatch update of the token-transformer policy:
forward -> PPO clipped loss fwd+bwd -> backward -> global-norm clip + Adam,
on B = 512 rows drawn (epoch permutations) from a 16 384-row synthetic
rollout resident in HBM.  Model: 96 entity tokens (+READOUT), 32 numeric
token features, card ids in [0, 2048), d 256 / 4 heads / FFN 1024 / 4 pre-LN
layers, 64 masked options, blind value head, fp32 throughout.

The step is captured once in a HIP graph (sync-free compact layout) and
replayed per minibatch with the minibatch's row indices written into the
captured index buffer, as the reference's trainer replays its captured train
graph; `value` is the throughput of those replays.  The same number of
minibatches then runs launched kernel by kernel, once with no launch profile
open (`stream_launch`: host row counts, weight gradients on a side stream)
and once with a HIP event pair around every GEMM / LayerNorm / Adam launch
(`profiled_pass`); the kernels' rooflines come from the latter (`--stream`
times only the stream-launched passes).

Prints one JSON line (see the keys below), including the GEMM kernel's
roofline (useful flops over measured kernel time, HIP events on the launch
stream) and the host-CPU baseline (the oracle: PyTorch CPU restatement of
the same step, timed on a bounded sample in the same run).

Secondary workloads (not the headline line): ``--workload rollout`` times
the rollout step — inference forward of 8192 rows plus one sampled action
per row; ``--workload frozen`` times the training step of the reference's
own model variant (frozen layout: 160 tokens, d256/H8/FFN512, static-table
card vectors, oracle critic over 218 positions, aux losses);
``--workload replay`` times the rollout-side steps around the training step
(negamax advantage, prioritized replay draw, train-layout transposes);
``--workload bf16`` times the training step at B = 2048 with the GEMMs' and
attention's products in bf16 (fp32 accumulation; everything else fp32).
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "PPO minibatch step obs/sec (fwd+bwd+Adam) @B=512; % MFMA/HBM roofline"
FP32_MFMA_PEAK_TFLOPS = 157.3      # MI355X dense fp32 matrix peak
BF16_MFMA_PEAK_TFLOPS = 2500.0     # MI355X dense bf16 matrix peak
HBM_PEAK_GBS = 8000.0              # MI355X HBM3E bandwidth
# launch classes of ptcg_profile_class: (index, name); amounts are HBM bytes
HBM_CLASSES = ((1, "layernorm_fwd"), (2, "layernorm_bwd"), (3, "adam_norm"), (4, "adam_update"),
               (7, "embedding_gather"), (8, "ppo_loss_softmax"))

TRAIN = dict(learning_rate=3e-4, beta1=0.9, beta2=0.999, eps=1e-8, max_grad_norm=0.5,
             clip_coef=0.2, vf_clip_coef=0.2, vf_coef=0.5, ent_coef=0.01)


PROFILED_NOTE = ("the same minibatches again with a HIP event pair around every GEMM / LayerNorm / Adam launch "
                 "and the blocks' weight gradients on the launch stream; roofline and hbm_kernels come from "
                 "this pass")


def option_rows(dm, obs_rows):
    """Option rows the loss can see: each row's legal options (all of them
    in a row with none legal); a masked option's score reaches the PPO loss
    only as the constant -1e4."""
    off = dm.offsets()
    mask = obs_rows[:, off["opt_mask"][0]:off["opt_mask"][1]] != 0
    legal = mask.sum(1)
    return float(np.where(legal > 0, legal, dm.n_opt).sum())


def useful_gemm_flops(dm, obs_rows):
    """Useful GEMM flops of one fwd+bwd over `obs_rows`: token rows count
    only valid tokens (+READOUT in the trunk), option rows only the options
    the loss can see; every GEMM's backward is 2x its forward (dX and dW),
    so fwd+bwd = 3x fwd."""
    from ptcg_amd.params import OPT_E, SC_H, VAL_H, DEC_H
    off = dm.offsets()
    zone = obs_rows[:, off["tok_int"][0]:off["tok_int"][1]].reshape(len(obs_rows), dm.l_tok, dm.tok_int)[:, :, 1]
    n_valid = (zone > 0).sum(1).astype(np.float64)
    Lv = n_valid + 1
    d, ffn, B = dm.d, dm.ffn, len(obs_rows)
    NJ = option_rows(dm, obs_rows)
    tok_in = 2 * dm.d_c + dm.tok_f + 12
    fwd = 2.0 * n_valid.sum() * tok_in * d
    fwd += dm.layers * (Lv.sum() * (8 * d * d + 4 * d * ffn))
    fwd += 2.0 * NJ * (dm.d_c * OPT_E + dm.d_a * OPT_E + dm.q_in * d + d * d + dm.score_in * SC_H)
    fwd += 2.0 * B * (dm.global_f * dm.g + dm.g * dm.g + dm.dec_in * DEC_H + DEC_H * DEC_H
                      + dm.bcast_in * d + dm.val_in * VAL_H)
    return 3.0 * fwd, float(Lv.mean())


def _gemm_list(dm, obs_rows):
    """(rows M, in K, out N, GELU epilogue, residual epilogue, trunk block
    product: 0 none, 1 QKV, 2 out-projection, 3 FFN1, 4 FFN2) of every linear
    layer of the forward, on valid rows only."""
    from ptcg_amd.params import OPT_E, SC_H, VAL_H, DEC_H
    off = dm.offsets()
    zone = obs_rows[:, off["tok_int"][0]:off["tok_int"][1]].reshape(len(obs_rows), dm.l_tok, dm.tok_int)[:, :, 1]
    n_valid = float((zone > 0).sum())
    R = n_valid + len(obs_rows)
    d, ffn, B = dm.d, dm.ffn, len(obs_rows)
    NJ = option_rows(dm, obs_rows)
    g = [(n_valid, 2 * dm.d_c + dm.tok_f + 12, d, 0, 0, 0)]
    for _ in range(dm.layers):
        g += [(R, d, 3 * d, 0, 0, 1), (R, d, d, 0, 1, 2), (R, d, ffn, 1, 0, 3), (R, ffn, d, 0, 1, 4)]
    g += [(NJ, dm.d_c, OPT_E, 0, 0, 0), (NJ, dm.d_a, OPT_E, 0, 0, 0), (NJ, dm.q_in, d, 1, 0, 0),
          (NJ, d, d, 0, 0, 0), (NJ, dm.score_in, SC_H, 1, 0, 0), (B, dm.global_f, dm.g, 1, 0, 0),
          (B, dm.g, dm.g, 0, 0, 0), (B, dm.dec_in, DEC_H, 1, 0, 0), (B, DEC_H, DEC_H, 0, 0, 0),
          (B, dm.bcast_in, d, 0, 0, 0), (B, dm.val_in, VAL_H, 1, 0, 0)]
    return g


def algorithmic_gemm_bytes(dm, obs_rows, bf16_blocks=False):
    """HBM bytes of one fwd+bwd's GEMMs with every operand read and every
    output written once: forward X, W, Y (+ GELU output, + residual read);
    backward dX = dY W (+ pre-activation read for a GELU input) and
    dW = dY^T X.  fp32 throughout, or (bf16_blocks) the bf16 variant's trunk
    blocks: bf16 activations, weight copies and backward operands, fp32
    residual stream (the residual epilogues' R and C), fp32 dX where a
    LayerNorm backward reads it (QKV and FFN1 dX) and fp32 weight gradients."""
    tot = 0.0
    for M, K, N, gelu, resid, trunk in _gemm_list(dm, obs_rows):
        if bf16_blocks and trunk:
            fwd = 2 * M * K + 2 * N * K + (8 * M * N if resid else (4 if gelu else 2) * M * N)
            # dX = dY W: dY bf16; output fp32 for the LayerNorm backward
            # (QKV, FFN1), bf16 for the attention backward (out-projection)
            # and for the GELU layer (FFN2, + the bf16 gelu'(z) read)
            dx = 2 * M * N + 2 * N * K + {1: 4, 2: 2, 3: 4, 4: 4}[trunk] * M * K
            dw = 2 * M * N + 2 * M * K + 4 * N * K
            tot += fwd + dx + dw
        else:
            fwd = M * K + N * K + M * N * (2 if gelu else 1) + (M * N if resid else 0)
            dx = M * N + N * K + M * K
            dw = M * N + M * K + N * K
            # the GELU backward reads the saved pre-activation in the dX
            # product of the layer after it (one extra M x N read per GELU layer);
            # a residual product at d = 256 also writes the LayerNorm of its
            # output (y, mean, rstd) in the same launch
            ln = M * N + 2 * M if resid and N == 256 else 0
            tot += 4.0 * (fwd + dx + dw + (M * N if gelu else 0) + ln)
    return tot


def gemm_source_sha():
    """sha256 (first 16 hex) of the GEMM kernel source the library was built from."""
    import hashlib
    with open(os.path.join(ROOT, "kaggle-ptcg-ai-battle_amd", "csrc", "gemm.hip"), "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:16]


def measured_gemm_traffic():
    """HBM bytes per GEMM launch measured with rocprofv3 --pmc (FETCH_SIZE,
    WRITE_SIZE, copy-kernel calibrated) for this workload, read from the
    committed profile summary, which records the sha256 of the gemm.hip it
    was measured on.  Returns (bytes or None, provenance note): None when the
    summary is absent or was measured on another gemm.hip (stale)."""
    import re
    rel = os.path.join("profiles", "ptcg_step_b512_fp32_gemm_hbm_traffic.md")
    try:
        txt = open(os.path.join(ROOT, rel)).read()
    except OSError:
        return None, f"{rel} absent"
    m = re.search(r"traffic_bytes_per_launch\s*\|\s*([0-9.e+]+)", txt)
    h = re.search(r"gemm_hip_sha256_16\s*\|\s*([0-9a-f]+)", txt)
    cur = gemm_source_sha()
    if not m or not h:
        return None, f"{rel} has no traffic figure with its gemm.hip sha"
    if h.group(1) != cur:
        return None, f"stale: {rel} was measured on gemm.hip {h.group(1)}, this build is {cur}"
    return float(m.group(1)), f"rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, {rel} (gemm.hip {cur})"


def hbm_kernels(L, K):
    """Achieved HBM bandwidth of the memory-bound kernels of the timed steps:
    algorithmic bytes (each launch's inputs read and outputs written once) over
    the summed HIP-event durations of their launches."""
    out = {}
    tot_ms, tot_b = 0.0, 0.0
    for cls, name in HBM_CLASSES:
        ms, n, amt = ctypes.c_double(), ctypes.c_int(), ctypes.c_double()
        native_check(L.ptcg_profile_class(cls, ctypes.byref(ms), ctypes.byref(n), ctypes.byref(amt)))
        if n.value == 0 or ms.value <= 0:
            continue
        gbs = amt.value / (ms.value / 1e3) / 1e9
        out[name] = dict(achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s", frac=round(gbs / HBM_PEAK_GBS, 4),
                         launches_per_step=n.value / K, avg_launch_us=round(ms.value * 1e3 / n.value, 2),
                         bytes_per_launch=round(amt.value / n.value))
        if name.startswith("adam"):
            tot_ms += ms.value
            tot_b += amt.value
    if tot_ms > 0:
        gbs = tot_b / (tot_ms / 1e3) / 1e9
        out["adam"] = dict(achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s", frac=round(gbs / HBM_PEAK_GBS, 4),
                           note="norm + update passes, 32 B per parameter")
    return out


def muon_stats(L, K):
    """The Muon step of the timed steps: whole-step time (event pair around
    its launches) and its Newton-Schulz GEMMs' rate."""
    out = {}
    for cls, name in ((5, "step"), (6, "ns_gemm")):
        ms, n, amt = ctypes.c_double(), ctypes.c_int(), ctypes.c_double()
        native_check(L.ptcg_profile_class(cls, ctypes.byref(ms), ctypes.byref(n), ctypes.byref(amt)))
        out[name + "_ms_per_step"] = round(ms.value / K, 4)
        out[name + "_launches_per_step"] = n.value / K
        if name == "ns_gemm" and ms.value > 0:
            out["ns_tflops"] = round(amt.value / (ms.value / 1e3) / 1e12, 3)
            out["ns_tflop_per_step"] = round(amt.value / K / 1e12, 5)
    return out


def native_check(rc):
    from ptcg_amd import native
    native.check(rc)


def cpu_baseline(dm, obs, inp, B, budget_s, warmup=3, timed=10):
    """Oracle (torch CPU, fp32) fwd+bwd+PPO+clip+Adam on B-row minibatches of
    the same rollout: `warmup` untimed steps, then the median of `timed`
    steps (more while under `budget_s` of timed CPU work).  Threads: the
    host's os.cpu_count(), unless OMP_NUM_THREADS sets the process's share
    (both are reported)."""
    import torch
    import oracle.model as om
    import oracle.adam as oa
    import oracle.step as ost
    host = os.cpu_count() or 1
    omp = os.environ.get("OMP_NUM_THREADS")
    threads = int(omp) if omp else host
    torch.set_num_threads(threads)
    ref = om.build(dm, seed=0)
    opt = oa.OracleAdam([p for _, p in ref.named_blob_params()], lr=TRAIN["learning_rate"])
    hyp = dict(TRAIN)
    rng = np.random.default_rng(0)
    times = []
    for k in range(warmup + 10 ** 6):
        idx = rng.choice(len(obs), B, replace=False)
        t0 = time.perf_counter()
        ost.minibatch_step(ref, opt, obs[idx], {k2: v[idx] for k2, v in inp.items()}, hyp)
        if k >= warmup:
            times.append(time.perf_counter() - t0)
        if len(times) >= timed and sum(times) > budget_s or len(times) >= 4 * timed:
            break
    med = float(np.median(times))
    return dict(value=B / med, unit="obs/s", cores=threads, kind="port", host_cpu_count=host,
                omp_num_threads=int(omp) if omp else None,
                sample=f"median of {len(times)} timed oracle minibatch steps of {B} rows after {warmup} warmup "
                       f"(fwd+bwd+PPO+clip+Adam, torch CPU fp32, {threads} threads), {med:.2f} s/step")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--minibatch", type=int, default=512)
    ap.add_argument("--rollout", type=int, default=16384)
    ap.add_argument("--cpu-seconds", type=float, default=20.0,
                    help="CPU baseline: keep timing past 10 steps while under this many seconds")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--workload", choices=("train", "rollout", "frozen", "bf16", "replay"), default="train")
    ap.add_argument("--rollout-rows", type=int, default=8192)
    ap.add_argument("--rollout-precision", choices=("fp32", "bf16"), default="fp32",
                    help="--workload rollout: fp32 or bf16 GEMM and attention products")
    ap.add_argument("--sampler", choices=("inverse_cdf", "gumbel"), default="gumbel",
                    help="--workload rollout: the action draw (Gumbel-max from counter-based noise, "
                         "or the reference's inverse CDF)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run three 256 MiB device-to-device copies (the HBM counter calibration)")
    ap.add_argument("--copy-rate", action="store_true",
                    help="only time device-to-device copies of the memory-bound kernels' sizes (GB/s for scale)")
    ap.add_argument("--optimizer", choices=("adam", "muon"), default="adam",
                    help="optimizer of the training step (muon: the reference's, secondary line)")
    ap.add_argument("--stream", action="store_true",
                    help="time stream launches only (default for the training step: HIP graph replay for the "
                         "value, then a stream-launched pass for the kernel rooflines)")
    ap.add_argument("--sync-free", action="store_true",
                    help="compact row count kept on the device (no host read-back per forward)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the data-parallel path is designed but not built)", file=sys.stderr)
        sys.exit(2)

    import __graft_entry__
    __graft_entry__.load_package()
    from ptcg_amd import dims, synth, trainer, native, devmem
    if args.copy_calibration:
        # a plain copy of known size: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of
        # this run give the counters' scale (bytes read / written per KiB counted)
        n = 64 << 20
        x = devmem.DeviceArray(n)
        native.check(native.lib().ptcg_fill(x.data_ptr(), n, 1.0, None))
        y = devmem.DeviceArray(n)
        for _ in range(3):
            y.copy_(x)
        devmem.synchronize()
        print(json.dumps({"copy_bytes": n * 4, "copies": 3}), flush=True)
        return
    if args.copy_rate:
        # what a plain streaming copy reaches at the step's kernel sizes:
        # 38 MB (one 37.4k x 256 fp32 activation), 60 MB, 256 MB
        out = {}
        for mb in (38.3, 60.5, 256.0):
            n = int(mb * 1e6) // 4
            x = devmem.DeviceArray(n)
            native.check(native.lib().ptcg_fill(x.data_ptr(), n, 1.0, None))
            y = devmem.DeviceArray(n)
            for _ in range(5):
                y.copy_(x)
            e0, e1 = devmem.Event(), devmem.Event()
            ts = []
            for _ in range(20):
                e0.record()
                y.copy_(x)
                e1.record()
                ts.append(e0.elapsed_ms(e1))
            ms = sorted(ts)[len(ts) // 2]
            out[f"{mb:g}MB"] = dict(median_us=round(ms * 1e3, 2), gbs=round(2 * n * 4 / (ms / 1e3) / 1e9, 1))
        print(json.dumps({"copy_rate": out}), flush=True)
        return

    if args.workload == "rollout":
        return bench_rollout(args)
    if args.workload == "replay":
        return bench_replay(args)
    dm = dims.FROZEN if args.workload == "frozen" else dims.CORE
    B, R = args.minibatch, args.rollout
    bf16 = args.workload == "bf16"
    if bf16 and B == 512:
        B = 2048   # the mixed-precision configuration's minibatch
    if args.workload == "frozen":
        R = min(R, 4096)
    obs = synth.make_obs(dm, R, seed=1)
    inp = synth.make_ppo_inputs(dm, obs, seed=2)
    static = synth.make_static(dm, 4) if dm.tables == 1 else None
    muon = args.optimizer == "muon"
    # Muon with the reference trainer's settings (native/train_native.py: momentum = beta1 0.95)
    tcfg = dict(TRAIN, minibatch_size=B, **(dict(optimizer="muon", beta1=0.95, learning_rate=0.02) if muon else {}))
    # graph replay for the CORE training step (needs the sync-free step)
    graph = args.workload == "train" and not args.stream
    pl = trainer.create_pufferl({"dims": dm, "train": tcfg, "seed": 0, "static": static,
                                 "precision": "bf16" if bf16 else "fp32", "sync_free": args.sync_free or graph})
    trainer.set_rollout(pl, obs, **inp)
    n_lists = args.warmup + args.steps
    lists = synth.minibatch_indices(R, B, n_lists, seed=3)
    d_lists = [pl.to_device(ix, np.int32) for ix in lists]
    r = pl.rollout

    for i in range(args.warmup):
        pl.step(r["obs"], d_lists[i], r)
    devmem.synchronize()
    L = native.lib()
    K = args.steps
    sec_graph = None
    if graph:
        # timed region 1 (`value`): the step captured once in a HIP graph over a
        # fixed index buffer, refreshed and replayed per minibatch -- the
        # reference trainer's launch mode (pufferlib.cu:2019-2140)
        idx_buf = devmem.DeviceArray(B, np.int32)
        idx_buf.copy_(d_lists[0])
        devmem.synchronize()
        pl.capture_step(r["obs"], idx_buf, r)
        t0 = time.perf_counter()
        for i in range(args.warmup, n_lists):
            idx_buf.copy_(d_lists[i])
            pl.replay_step()
        devmem.synchronize()
        sec_graph = time.perf_counter() - t0
    # timed region 2 (the only one with --stream): the same number of
    # minibatches launched kernel by kernel, a HIP event pair on the launch
    # stream around every GEMM, LayerNorm and Adam launch -- the kernels'
    # rooflines.  While the profile is open the blocks' weight gradients stay
    # on the launch stream (no side stream), so no timed launch shares the
    # GPU with another.  Host row counts here, so every launch is sized exactly and
    # its algorithmic amount is the work it does (a sync-free launch covers
    # all N * l_seq rows and stops at the device count).
    if graph and not args.sync_free:
        native.check(L.ptcg_trainer_set_sync_free(pl._h, 0))
    sec_plain = None
    if not graph or args.workload == "train":
        # the value of a stream-launched workload (beside the graph replay's
        # for the CORE step): the minibatches launched kernel by kernel with
        # no launch profile open (the blocks' weight gradients on their side
        # stream); the profiled pass below repeats them
        if graph:   # one untimed step in host-row-count mode first
            pl.step(r["obs"], d_lists[0], r)
            devmem.synchronize()
        t0 = time.perf_counter()
        for i in range(args.warmup, n_lists):
            pl.step(r["obs"], d_lists[i], r)
        devmem.synchronize()
        sec_plain = time.perf_counter() - t0
    native.check(L.ptcg_profile_begin(256 * args.steps))
    t0 = time.perf_counter()
    for i in range(args.warmup, n_lists):
        pl.step(r["obs"], d_lists[i], r)
    devmem.synchronize()
    t1 = time.perf_counter()
    ms, launches, exec_flops = ctypes.c_double(), ctypes.c_int(), ctypes.c_double()
    native.check(L.ptcg_profile_end(ctypes.byref(ms), ctypes.byref(launches), ctypes.byref(exec_flops)))
    losses = trainer.log(pl)
    if not np.isfinite(losses["loss"].get("total", np.nan)):
        raise RuntimeError(f"non-finite loss during the benchmark: {losses}")

    sec_stream = t1 - t0
    sec = sec_graph if graph else sec_plain
    if args.workload == "frozen":
        line = {
            "metric": "PPO minibatch step obs/sec (fwd+bwd+Adam), reference model variant @B=512",
            "value": round(B * K / sec, 2), "unit": "obs/s", "n_gpus": 1, "steps": K, "warmup": args.warmup,
            "ms_per_step": round(sec * 1e3 / K, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
            "config": {"workload": "PPO minibatch step of the reference model variant: 160 tokens + READOUT, "
                                   "56 token features, d256/H8/FFN512/4 layers, static-table card vectors "
                                   "(1284 cards, 1573 attacks, 448 skills), oracle critic over 218 positions, "
                                   "blind-value / hand / prize aux losses",
                       "minibatch": B, "rollout_rows": R, "seq_len": dm.l_tok + 1, "parallelism": "single GPU"},
            "gemm": {"launches_per_step": launches.value / K, "gemm_ms_per_step": round(ms.value / K, 4),
                     "executed_tflops": round(exec_flops.value / (ms.value / 1e3) / 1e12, 3)},
            "hbm_kernels": hbm_kernels(L, K),
            "losses": {k: round(v, 5) for k, v in losses.items() if isinstance(v, float)},
            "profiled_pass": dict(value=round(B * K / sec_stream, 2), ms_per_step=round(sec_stream * 1e3 / K, 4),
                                  note=PROFILED_NOTE),
        }
        pl.close()
        print(json.dumps(line), flush=True)
        return
    useful = 0.0
    abytes = 0.0
    lv = []
    for ix in lists[args.warmup:]:
        f, l = useful_gemm_flops(dm, obs[ix])
        useful += f
        abytes += algorithmic_gemm_bytes(dm, obs[ix], bf16_blocks=bf16)
        lv.append(l)
    gemm_s = ms.value / 1e3
    achieved = useful / gemm_s / 1e12
    peak = BF16_MFMA_PEAK_TFLOPS if bf16 else FP32_MFMA_PEAK_TFLOPS
    traffic = measured_gemm_traffic()
    kname = ("gemm_bs32_kernel + gemm_bs_dw_kernel + gemm_resid_ln_kernel + gemm_dx_lnbwd_kernel (trunk blocks, "
             "bf16 operands) + gemm_bf16_k16_kernel"
             if bf16 else "gemm_f32_dma_kernel + gemm_f32_kernel + gemm_resid_ln_kernel")
    roof = dict(bound="mfma", kernel=f"{kname} (all launches: trunk, token, option and head GEMMs)",
                achieved=round(achieved, 3), peak=peak, unit="TFLOP/s",
                frac=round(achieved / peak, 4),
                traffic=None if bf16 else traffic[0], traffic_source=None if bf16 else traffic[1],
                algorithmic_bytes_per_launch=round(abytes / max(launches.value, 1)),
                launches_per_step=launches.value / K,
                avg_launch_us=round(ms.value * 1e3 / max(launches.value, 1), 3),
                gemm_ms_per_step=round(ms.value / K, 4),
                executed_tflops=round(exec_flops.value / gemm_s / 1e12, 3),
                useful_tflop_per_step=round(useful / K / 1e12, 4),
                mean_valid_seq=round(float(np.mean(lv)), 2))
    if not bf16 and dm.d == 256:
        roof["fused_layernorm"] = ("the blocks' residual products (out-projection, FFN2) run the LayerNorm that "
                                   "reads their output in the same launch (gemm_resid_ln_kernel): its time and "
                                   "its output bytes are inside these figures")
    if bf16 and dm.d == 256:
        roof["fused_layernorm"] = ("the bf16 blocks' residual products run the LayerNorm forward that reads their "
                                   "output (gemm_resid_ln_kernel), and their QKV / FFN1 dX products the LayerNorm "
                                   "backward that reads theirs (gemm_dx_lnbwd_kernel), in the same launch: those "
                                   "LayerNorms' time is inside these figures, their flops are not counted")
    if bf16:
        # The products' arithmetic intensity (useful flops over the operand /
        # output bytes: bf16 in the trunk blocks, fp32 residual stream and
        # elsewhere) is below the bf16 ridge point (peak flops / peak
        # bandwidth = 312 flop/B): the bf16 GEMMs are HBM-bound, so the
        # bound roofline is bytes over time; the MFMA fraction stays beside it.
        gbs = abytes / gemm_s / 1e9
        roof.update(bound="hbm", achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(gbs / HBM_PEAK_GBS, 4), mfma_tflops=round(achieved, 3), mfma_peak=peak,
                    mfma_frac=round(achieved / peak, 4), intensity_flop_per_byte=round(useful / abytes, 1),
                    ridge_flop_per_byte=round(peak * 1e12 / (HBM_PEAK_GBS * 1e9), 1))
    line = {
        "metric": ("PPO minibatch step obs/sec (fwd+bwd+Muon) @B=512" if muon else METRIC) if not bf16
                  else "PPO minibatch step obs/sec (fwd+bwd+Adam) @B=2048, bf16 GEMM and attention products",
        "value": round(B * K / sec, 2), "unit": "obs/s", "n_gpus": 1,
        "steps": K, "warmup": args.warmup, "ms_per_step": round(sec * 1e3 / K, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16" if bf16 else "fp32",
        "data": "synthetic",
        "config": {"workload": f"PPO minibatch step (fwd+bwd+PPO loss+grad-norm clip+Adam) on {B} rows of "
                               "a 16384-row HBM-resident rollout; 96 tokens + READOUT, 32 token features, "
                               "card ids [0,2048), d256/H4/FFN1024/4 layers, 64 options, blind value head"
                               + ("; bf16 GEMM and attention operands, fp32 accumulation, LayerNorm, "
                                  "softmax, loss, master weights and Adam state" if bf16 else ""),
                   "minibatch": B, "rollout_rows": R, "seq_len": dm.l_tok + 1,
                   "parallelism": "single GPU",
                   "compact_rows": "device count, no host read-back" if (args.sync_free or graph)
                   else "host read-back",
                   "launch": "HIP graph replay (step captured once)" if graph else "stream"},
        "roofline": roof,
        "hbm_kernels": hbm_kernels(L, K),
        "losses": {k: round(v, 5) for k, v in losses.items() if isinstance(v, float)},
    }
    if not graph:
        line["profiled_pass"] = dict(value=round(B * K / sec_stream, 2), ms_per_step=round(sec_stream * 1e3 / K, 4),
                                     note=PROFILED_NOTE)
    if graph:
        line["stream_launch"] = dict(value=round(B * K / sec_plain, 2), ms_per_step=round(sec_plain * 1e3 / K, 4),
                                     note="as many minibatches launched kernel by kernel (host row counts read "
                                          "back per minibatch, exact launch sizes, no launch profile open), the "
                                          "blocks' weight gradients on their side stream beside the dX chain")
        line["profiled_pass"] = dict(value=round(B * K / sec_stream, 2), ms_per_step=round(sec_stream * 1e3 / K, 4),
                                     note="as many minibatches launched kernel by kernel (host row counts, exact "
                                          "launch sizes) with HIP event pairs, the blocks' weight gradients on "
                                          "the launch stream so that every timed launch runs alone; roofline "
                                          "and hbm_kernels come from this pass")
    if muon:
        line["muon"] = muon_stats(L, K)
    if not args.no_cpu_baseline and not bf16:
        line["cpu_baseline"] = cpu_baseline(dm, obs, inp, B, args.cpu_seconds)
        line["gpu_over_cpu"] = round(line["value"] / line["cpu_baseline"]["value"], 1)
    pl.close()
    print(json.dumps(line), flush=True)


def bench_rollout(args):
    """Rollout step: inference forward of n rows (one block's activations
    reused across layers) + one sampled action per row (counter RNG)."""
    from ptcg_amd import dims, synth, trainer, native, devmem
    dm = dims.CORE
    n = args.rollout_rows
    obs = synth.make_obs(dm, n, seed=1)
    graph = not args.stream
    bf = args.rollout_precision == "bf16"
    pl = trainer.create_pufferl({"dims": dm, "train": dict(TRAIN, minibatch_size=8), "seed": 0,
                                 "sync_free": args.sync_free or graph, "precision": args.rollout_precision,
                                 "sampler": args.sampler})
    d_obs = pl.to_device(obs)
    for i in range(args.warmup):
        pl.rollout_step(d_obs, n, seed=0, step=i)
    devmem.synchronize()
    L = native.lib()
    K = args.steps
    sec_graph = None
    if graph:
        # timed region 1 (`value`): the rollout step captured once (a slot of
        # the reference's per-(t, buf) graphs) and replayed, the draw's step
        # advancing in a device counter
        outs = [devmem.DeviceArray(n) for _ in range(3)]
        step_dev = devmem.DeviceArray.from_numpy(np.array([args.warmup], np.int64))
        pl.capture_rollout(0, d_obs, n, 0, step_dev, *outs)
        t0 = time.perf_counter()
        for i in range(args.steps):
            pl.replay_rollout(0)
        devmem.synchronize()
        sec_graph = time.perf_counter() - t0
        if not np.isfinite(outs[1].numpy()).all():
            raise RuntimeError("non-finite log-probabilities in the rollout benchmark")
        transport = bench_transport(pl, dm, obs, n, args)
        native.check(L.ptcg_trainer_set_sync_free(pl._h, 0))   # exact launch sizes for the timing pass
    # timed region 2: launched call by call with HIP event pairs (the roofline)
    native.check(L.ptcg_profile_begin(256 * args.steps))
    t0 = time.perf_counter()
    for i in range(args.steps):
        acts, lps, vals = pl.rollout_step(d_obs, n, seed=0, step=args.warmup + i)
    devmem.synchronize()
    t1 = time.perf_counter()
    ms, launches, exec_flops = ctypes.c_double(), ctypes.c_int(), ctypes.c_double()
    native.check(L.ptcg_profile_end(ctypes.byref(ms), ctypes.byref(launches), ctypes.byref(exec_flops)))
    if not np.isfinite(lps.numpy()).all():
        raise RuntimeError("non-finite log-probabilities in the rollout benchmark")
    sec_stream = t1 - t0
    sec = sec_graph if graph else sec_stream
    useful, lv = useful_gemm_flops(dm, obs)
    useful_fwd = useful / 3.0
    gemm_s = ms.value / 1e3
    achieved = useful_fwd * K / gemm_s / 1e12
    line = {
        "metric": "rollout forward + action sampling obs/sec @8192 rows" + (", bf16 products" if bf else ""),
        "value": round(n * K / sec, 2),
        "unit": "obs/s", "n_gpus": 1, "steps": K, "warmup": args.warmup, "ms_per_step": round(sec * 1e3 / K, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16" if bf else "fp32", "data": "synthetic",
        "config": {"workload": f"inference forward of {n} obs rows (CORE model: 96 tokens + READOUT, d256/H4/"
                               "FFN1024/4 layers) + one action per row, "
                               + ("Gumbel-max over 64 options with Philox4x32-10 noise keyed (seed, step, row, option)"
                                  if args.sampler == "gumbel" else "inverse-CDF draw from Philox4x32-10"),
                   "sampler": args.sampler,
                   "rows": n, "seq_len": dm.l_tok + 1, "parallelism": "single GPU",
                   "launch": "HIP graph replay (step captured once)" if graph else "stream"},
        "roofline": dict(bound="mfma", kernel=("gemm_bf16_k16_kernel" if bf else "gemm_f32_dma_kernel + gemm_f32_kernel")
                         + " (forward GEMMs)", achieved=round(achieved, 3),
                         peak=BF16_MFMA_PEAK_TFLOPS if bf else FP32_MFMA_PEAK_TFLOPS, unit="TFLOP/s",
                         frac=round(achieved / (BF16_MFMA_PEAK_TFLOPS if bf else FP32_MFMA_PEAK_TFLOPS), 4),
                         traffic=None, gemm_ms_per_step=round(ms.value / K, 4),
                         launches_per_step=launches.value / K, mean_valid_seq=round(lv, 2)),
    }
    if graph:
        line["stream_launch"] = dict(value=round(n * K / sec_stream, 2), ms_per_step=round(sec_stream * 1e3 / K, 4),
                                     note="as many steps launched call by call (host row counts); the roofline "
                                          "comes from this pass")
        line["transport"] = transport
    pl.close()
    print(json.dumps(line), flush=True)


def bench_transport(pl, dm, obs, n, args):
    """PCIe-inclusive rollout rate through the pinned transport (vecenv.h GPU
    mode): the n agents split into two env buffers, each on its own rollout
    policy (activations), stream and draw-step counter; per step both
    buffers' captured rollout graphs and action downloads are launched, then
    each buffer's checked stream sync is followed by the async H2D of its
    observations, rewards and terminals, which overlaps the other buffer's
    work.  Not `value`: the observations cross PCIe here."""
    from ptcg_amd import transport as tr, devmem
    nbuf = 2
    x = tr.RolloutTransport(n, nbuf, dm.obs_size)
    try:
        x.observations[:] = obs
        step_dev = [devmem.DeviceArray(1, np.int64) for _ in range(nbuf)]
        for b in range(nbuf):
            x.capture_rollout(pl, b, 1 + b, 0, step_dev[b])   # slots 1, 2
        for b in range(nbuf):
            x.upload(b)

        def step():
            for b in range(nbuf):
                x.launch(pl, b, 1 + b)
            for b in range(nbuf):
                x.wait(b)
                x.upload(b)

        for _ in range(2):   # warm the slots
            step()
        devmem.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        devmem.synchronize()
        sec = time.perf_counter() - t0
        if not np.isfinite(x.actions).all():
            raise RuntimeError("non-finite actions in the transport benchmark")
        h2d = x.observations.nbytes + x.rewards.nbytes + x.terminals.nbytes
        return dict(value=round(n * args.steps / sec, 2), unit="obs/s", buffers=nbuf,
                    ms_per_step=round(sec * 1e3 / args.steps, 4), h2d_bytes_per_step=int(h2d),
                    d2h_bytes_per_step=int(x.actions.nbytes),
                    note="pinned host observations up and actions down per env buffer around the captured "
                         "rollout graphs, buffers' forwards in flight together (PCIe-inclusive; the env step "
                         "itself is not run)")
    finally:
        x.close()


def bench_replay(args):
    """Rollout-side steps of train_impl at the reference trainer's defaults
    (native/train_native.py: total_agents 2048, horizon 64, minibatch 1024):
    per minibatch the negamax advantage over the whole rollout and one
    prioritized draw of 16 segments (weights, row indices); per epoch the
    transposes of the rollout into the train layout (obs rows of the CORE
    dims and the six per-step arrays).  Synthetic device data."""
    from ptcg_amd import dims, native, devmem
    import oracle.replay as orp
    L = native.lib()
    dm = dims.CORE
    W, S, T, mb = dm.obs_size, 2048, 64, 1024
    n, segs, seat = S * T, mb // T, dm.seat_col()
    rng = np.random.default_rng(5)
    # obs rows: only the seat column is read by the advantage (the transposes
    # move whatever bytes are there), so the rest stays zero
    seat_col = rng.integers(0, 2, n).astype(np.float32)
    obs_host = np.zeros((n, W), np.float32)
    obs_host[:, seat] = seat_col
    obs_tb = devmem.DeviceArray.from_numpy(obs_host)
    del obs_host
    obs = devmem.DeviceArray(n * W)
    D = devmem.DeviceArray.from_numpy
    small_tb = [D(rng.standard_normal(n).astype(np.float32)) for _ in range(6)]
    small = [devmem.DeviceArray(n) for _ in range(6)]
    values_h = rng.standard_normal(n).astype(np.float32)
    rewards_h = (rng.random(n) * 2 - 1).astype(np.float32)
    dones_h = (rng.random(n) < 0.02).astype(np.float32)
    ratio_h = (rng.random(n) + 0.5).astype(np.float32)
    values, rewards, dones, ratio = D(values_h), D(rewards_h), D(dones_h), D(ratio_h)
    adv, ret = devmem.DeviceArray(n), devmem.DeviceArray(n)
    probs, cdf, mbp = devmem.DeviceArray(S), devmem.DeviceArray(S), devmem.DeviceArray(segs)
    idx, rows = devmem.DeviceArray(segs, np.int32), devmem.DeviceArray(mb, np.int32)
    rprio, off = devmem.DeviceArray(n), devmem.DeviceArray(1, np.int64)
    P = lambda t: t.data_ptr()

    def transposes():
        native.check(L.ptcg_transpose_102(P(obs), P(obs_tb), T, S, W, 0, None))
        for k in range(6):
            native.check(L.ptcg_transpose_102(P(small[k]), P(small_tb[k]), T, S, 1, int(k == 1), None))

    def advantage():
        native.check(L.ptcg_negamax_advantage(P(values), P(rewards), P(dones), P(ratio), P(obs), W, seat, P(adv),
                                              P(ret), 1.0, 0.95, 1.0, 1.0, S, T, None))

    def replay():
        native.check(L.ptcg_prio_replay(P(adv), S, T, 0.8, segs, S, 0.2, 7, P(off), P(probs), P(cdf), P(idx),
                                        P(mbp), P(rows), P(rprio), None))

    def timed(fn, reps):
        for _ in range(3):
            fn()
        devmem.synchronize()
        ev = [(devmem.Event(), devmem.Event()) for _ in range(reps)]
        for a, b in ev:
            a.record()
            fn()
            b.record()
        devmem.synchronize()
        return sorted(a.elapsed_ms(b) for a, b in ev)[reps // 2] * 1e3   # median us

    K = args.steps
    t_obs = timed(lambda: native.check(L.ptcg_transpose_102(P(obs), P(obs_tb), T, S, W, 0, None)), max(5, K // 4))
    t_tr = timed(transposes, max(5, K // 4))
    t_adv = timed(advantage, K)
    t_rep = timed(replay, K)
    # whole minibatch prep, back to back (advantage then replay), K times
    devmem.synchronize()
    t0 = time.perf_counter()
    for _ in range(K):
        advantage()
        replay()
    devmem.synchronize()
    sec = time.perf_counter() - t0
    obs_bytes = 2.0 * n * W * 4
    adv_bytes = n * (4 * 4 + 4 + 2 * 4)        # values, rewards, dones, ratio, seat; advantages, returns
    line = {
        "metric": "rollout-side minibatch prep (negamax advantage + prioritized replay draw) per second "
                  "@2048 segments x 64 steps, minibatch 1024",
        "value": round(K / sec, 2), "unit": "minibatches/s", "n_gpus": 1, "steps": K, "warmup": 3,
        "ms_per_step": round(sec * 1e3 / K, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32", "data": "synthetic",
        "config": {"workload": "train_impl's per-minibatch rollout-side work at total_agents 2048, horizon 64, "
                               "minibatch 1024 (16 segments), CORE obs rows (4736 floats); per-epoch transposes "
                               "(T, B, ...) -> (B, T, ...)", "segments": S, "horizon": T, "minibatch": mb},
        # event pairs around each host call: the short kernels' figures include
        # the host's launch gap (the GPU idles between calls); kernel-only
        # durations come from a rocprofv3 kernel trace of this workload
        "per_call_us_host_inclusive": {"negamax_advantage": round(t_adv, 2), "prio_replay": round(t_rep, 2),
                                       "transpose_obs": round(t_obs, 1), "epoch_transposes": round(t_tr, 1)},
        "roofline": dict(bound="hbm", kernel="transpose_rows_kernel (obs rows into the train layout, per epoch)",
                         achieved=round(obs_bytes / (t_obs / 1e6) / 1e9, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                         frac=round(obs_bytes / (t_obs / 1e6) / 1e9 / HBM_PEAK_GBS, 4), traffic=None,
                         bytes_per_launch=obs_bytes),
        "advantage_bytes_per_launch": adv_bytes,
    }
    if not args.no_cpu_baseline:
        # the oracle's numpy restatement on the host: advantage + replay draw
        # the same arrays, in the train layout the advantage reads
        v, rr, dd, ii = (a.reshape(S, T) for a in (values_h, rewards_h, dones_h, ratio_h))
        st = seat_col.reshape(T, S).T.copy()    # obs rows after the (T, S) -> (S, T) transpose
        reps, t0 = 0, time.perf_counter()
        while True:
            a, _ = orp.negamax_advantage(v, rr, dd, ii, st, 1.0, 0.95, 1.0, 1.0)
            orp.prio_replay(a, 0.8, segs, S, 0.2, 7, 0)
            reps += 1
            if time.perf_counter() - t0 > min(args.cpu_seconds, 10.0) and reps >= 2:
                break
        cs = (time.perf_counter() - t0) / reps
        line["cpu_baseline"] = dict(value=round(1.0 / cs, 3), unit="minibatches/s", cores=1, kind="port",
                                    sample=f"{reps} minibatch preps (numpy, vectorized over segments)")
        line["gpu_over_cpu"] = round(line["value"] / line["cpu_baseline"]["value"], 1)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
