"""The drop-in boundary on the CPU: the mirror of ``_C.log`` against the key
accesses the reference's driver makes (native/train_native.py:660-757), the
PtcgLog struct against the C header, the integration guide's optimizer
binding against the package's own declaration, and a product path free of
torch."""
import ctypes
import math
import os
import re
import subprocess
import sys
import types

import numpy as np
import pytest

from ptcg_amd import native, trainer

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _fake_pl(global_step, epoch, last_step, last_time, start):
    return types.SimpleNamespace(global_step=global_step, epoch=epoch, _last_log_step=last_step,
                                 _last_log_time=last_time, _start_time=start)


def _log_struct(n=4.0, kl_skipped=3.0, vf_skipped=1.0):
    st = native.CPtcgLog()
    for i, v in enumerate((0.4, 2.0, 4.8, 1.2, 0.02, 0.06, 0.5)):
        st.loss[i] = v
    st.n, st.kl_skipped, st.vf_skipped, st.gate = n, kl_skipped, vf_skipped, 0.0
    st.grad_norm, st.lr, st.ent_coef, st.gpu_percent = 0.75, 3e-4, 0.01, 87.0
    for i in range(native.PERF_N):
        st.perf_s[i] = 0.5 * (i + 1)
    st.vram_used_gb, st.vram_total_gb = 12.5, 288.0
    st.global_step, st.epoch = 16384, 3
    return st


def test_log_serves_the_reference_driver():
    """Every access native/train_native.py makes on ``_C.log(pl)`` (its
    progress print, the divergence guard and the wandb row) succeeds on the
    mirror's dictionary and reads the values the trainer holds."""
    pl = _fake_pl(16384, 3, 0, 100.0, 90.0)
    logs = trainer.log_dict(pl, _log_struct(), now=102.0)
    # the progress line (train_native.py:662-684)
    env = logs.get("env", {})
    loss = logs.get("loss", {})
    line = (f"SPS {logs['SPS']} lr {logs.get('lr', 1.0):.5f} vram {logs['util']['vram_used_gb']:.1f}G "
            f"win_vs_rand {env.get('win_vs_rand', -1):.3f} ent {loss.get('entropy', 0):.3f} "
            f"kl {loss.get('kl', 0):.4f} vf {loss.get('value', 0):.4f} "
            f"klskip {loss.get('kl_skipped', 0):.0f} vfskip {loss.get('vf_skipped', 0):.0f}")
    assert "klskip 3 vfskip 1" in line and "vram 12.5G" in line
    # the divergence guard (:698-734) reads real numbers, so it can fire
    kl, vfl = loss.get("kl"), loss.get("value")
    assert kl is not None and vfl is not None
    bad = [k for k in ("kl", "entropy", "total", "value") if (v := loss.get(k)) is not None and not math.isfinite(v)]
    assert bad == []
    # the wandb row (:739-757)
    flat = {"SPS": logs["SPS"], "agent_steps": logs["agent_steps"], "epoch": 3, "lr": logs.get("lr", 1.0)}
    flat.update({f"losses/{k}": v for k, v in loss.items()})
    assert flat["agent_steps"] == 16384 and flat["SPS"] == 16384 // 2
    assert set(loss) == {"policy", "value", "entropy", "total", "old_kl", "kl", "clipfrac", "kl_skipped",
                         "vf_skipped"}
    # values: sums * (1/n) in fp32 (bindings.cu:59-66), applied lr, the counters
    inv = np.float32(1.0) / np.float32(4.0)
    assert loss["kl"] == float(np.float32(np.float32(0.06) * inv))
    assert loss["policy"] == float(np.float32(np.float32(0.4) * inv))
    assert abs(logs["lr"] - 3e-4) < 1e-10 and logs["epoch"] == 3
    assert logs["perf"]["train"] == logs["perf"]["train_misc"] + logs["perf"]["train_forward"]
    assert set(logs["perf"]) >= {"rollout", "eval_gpu", "eval_env", "train_misc", "train_forward", "train"}
    assert logs["util"]["gpu_percent"] == 87.0 and abs(logs["util"]["gpu_mem"] - 100 * 12.5 / 288) < 1e-9
    assert logs["minibatches"] == 4 and logs["grad_norm"] == 0.75


def test_log_without_minibatches_has_an_empty_loss_dict():
    """As the reference's: no minibatch since the last log -> ``loss`` is
    empty and the driver's ``.get`` defaults apply; SPS follows the steps
    since the last log."""
    pl = _fake_pl(100, 1, 100, 50.0, 40.0)
    logs = trainer.log_dict(pl, _log_struct(n=0.0), now=60.0)
    assert logs["loss"] == {} and logs["SPS"] == 0
    assert logs.get("loss", {}).get("kl", 0) == 0
    pl.global_step = 1100
    logs = trainer.log_dict(pl, _log_struct(n=0.0), now=70.0)
    assert logs["SPS"] == 100                       # 1000 steps over 10 s
    logs = trainer.log_dict(pl, _log_struct(n=0.0), now=70.0, reset=False)
    assert logs["SPS"] == 0                         # dt = 0 after the reset above


def test_log_struct_matches_the_header(tmp_path):
    """struct PtcgLog's size and field offsets from the C header (compiled
    with gcc) equal the ctypes declaration the mirror reads it through."""
    fields = ["loss", "n", "kl_skipped", "vf_skipped", "gate", "grad_norm", "lr", "ent_coef", "gpu_percent",
              "perf_s", "vram_used_gb", "vram_total_gb", "global_step", "epoch"]
    src = tmp_path / "layout.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "ptcg_amd.h"\nint main(void) {\n'
                   '  printf("size %zu\\n", sizeof(PtcgLog));\n'
                   + "".join(f'  printf("{f} %zu\\n", offsetof(PtcgLog, {f}));\n' for f in fields)
                   + '  printf("perf_n %d\\n", PTCG_PERF_N);\n  return 0;\n}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = dict(l.split() for l in subprocess.run([str(exe)], capture_output=True, text=True,
                                                 check=True).stdout.splitlines())
    assert int(got["size"]) == ctypes.sizeof(native.CPtcgLog)
    assert int(got["perf_n"]) == native.PERF_N
    for f in fields:
        assert int(got[f]) == getattr(native.CPtcgLog, f).offset, f


def test_integration_adam_binding_matches_the_package():
    """The integration guide's ctypes example binds ptcg_adam_step / _lrf with
    the argument types native.py declares (lr a device pointer, not a
    double).  The example's list expression ([ctypes.X] * k + ...) is read
    term by term."""
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    m = re.search(r"^ADAM_ARGTYPES = (.*?)\n(?=\S)", doc, flags=re.S | re.M)
    assert m, "the integration guide has no ADAM_ARGTYPES binding"
    argtypes = []
    for name, k in re.findall(r"\[ctypes\.(\w+)\](?:\s*\*\s*(\d+))?", m.group(1)):
        argtypes += [getattr(ctypes, name)] * int(k or 1)
    for name in ("ptcg_adam_step", "ptcg_adam_step_lrf"):
        assert argtypes == native._SIGS[name][1], name
        assert f"lib.{name}.argtypes = ADAM_ARGTYPES" in doc
    assert native._SIGS["ptcg_adam_step"][1][5] is ctypes.c_void_p     # lr: const double*


def test_gate_counters_in_the_oracle():
    """The two skip counters' rule (pufferlib.cu:1299-1301): every veto
    counts once in kl_skipped; vf_skipped counts the vetoes whose value test
    failed, whatever the KL test said."""
    from oracle import ppo as oppo
    cases = [(0.01, 0.1, 0.05, 0.5), (0.06, 0.1, 0.05, 0.5), (0.01, 0.7, 0.05, 0.5), (0.06, 0.7, 0.05, 0.5),
             (float("nan"), 0.1, 0.05, 0.5), (0.01, float("inf"), 0.0, 0.5)]
    want = [(0, 0), (1, 0), (1, 1), (1, 1), (1, 0), (1, 1)]
    for (kl, vf, kt, vt), (ks, vs) in zip(cases, want):
        gate = oppo.kl_gate(kl, vf, kt, vt)
        assert 1.0 - gate == ks
        assert 1.0 - oppo.kl_gate(kl, vf, 0.0, vt) == vs


def test_product_path_imports_no_torch():
    """The trainer mirror, the device-memory helpers and the transport load
    without torch: device memory goes through the library's C ABI."""
    code = ("import sys; sys.path.insert(0, %r); import __graft_entry__ as g; g.load_package(); "
            "import ptcg_amd.trainer, ptcg_amd.devmem, ptcg_amd.transport, ptcg_amd.native; "
            "assert 'torch' not in sys.modules, 'torch imported'" % ROOT)
    subprocess.run([sys.executable, "-c", code], check=True, timeout=120)
