"""Host-side mirror of the reference trainer's Python API for the training
step (the ``_C`` module of native/src/bindings.cu:675-862 as used by
native/train_native.py and native/tools/model_parity.py).

Same names, argument meaning and error behaviour (``RuntimeError`` with the
reference's messages) for the hot-path subset:

    create_pufferl(args) -> PuffeRL         bindings.cu:581-673
    train(pl) -> dict                       bindings.cu:184-192 / train_impl
                                            (segment rollouts: advantage ->
                                            prioritized replay -> step ->
                                            ratio / value write-back)
    debug_forward(pl, rows) -> (B, A+1)     bindings.cu:221-250
    save_weights / load_weights             bindings.cu:202-215, 339-367
    save_state / load_state                 bindings.cu:257-337 (Adam state)
    log(pl) -> dict                         bindings.cu:15-118 ("losses")
    close(pl)

Rollout collection is out of scope: ``set_rollout`` hands the trainer a
device-resident rollout (obs rows plus per-row actions, old log-probs,
advantages, returns, old values) in place of the env/vec pipeline, trained
from index lists; ``set_segment_rollout`` hands it what the reference's
trainer holds after collection (total_agents segments of horizon steps:
obs, actions, log-probs, rewards, terminals, values), and ``train`` then runs
train_impl's minibatch loop (pufferlib.cu:1963-2160) on the device.
Device memory for the rollout is plumbing held in torch tensors; every
computation runs in libptcg_amd.so.
"""
import ctypes

import numpy as np

from . import dims as dims_mod
from .native import lib, check, fptr, CPtcgHypers, c_void_p, c_i32_p

LOSS_KEYS = ("policy_loss", "value_loss", "entropy", "total_loss",
             "old_approx_kl", "approx_kl", "clipfrac")

TRAIN_DEFAULTS = {
    "learning_rate": 3e-4, "beta1": 0.9, "beta2": 0.999, "eps": 1e-8,
    "max_grad_norm": 0.5, "clip_coef": 0.2, "vf_clip_coef": 0.2,
    "vf_coef": 0.5, "ent_coef": 0.01, "kl_skip_threshold": 0.0,
    "vf_skip_threshold": 0.0, "minibatch_size": 512, "update_epochs": 4,
    "minibatches_per_epoch": 8,
    # segment rollouts (train_impl; native/train_native.py:250-270 values)
    "gamma": 1.0, "gae_lambda": 0.95, "vtrace_rho_clip": 1.0, "vtrace_c_clip": 1.0,
    "prio_alpha": 0.8, "prio_beta0": 0.2, "replay_ratio": 1.0, "total_epochs": 1,
    # "adam" (clip + Adam) or "muon" (the reference's optimizer: momentum = beta1,
    # decoupled weight decay muon_wd_1d on 1-D tensors)
    "optimizer": "adam", "muon_wd_1d": 0.0,
    # per-epoch schedules of train_impl (pufferlib.cu:1912-1948; train_native.py
    # build_args keys).  Off by default: the benchmark configs train at a fixed lr.
    "anneal_lr": 0, "min_lr_ratio": 0.0, "lr_warmup_epochs": 0, "start_epoch": 0,
    "lr_anneal_from_epoch": 0, "anneal_ent_coef": 0, "min_ent_coef_ratio": 0.1,
}


def _f32(x):
    return float(np.float32(x))


def cosine_annealing(base, lo, t, T):
    """pufferlib.cu:1828-1833: lo + (base - lo)(1 + cos(pi t/T))/2, fp32 result."""
    if T == 0:
        return _f32(base)
    ratio = min(1.0, max(0.0, _f32(t / T)))
    return _f32(_f32(lo) + 0.5 * _f32(_f32(base) - _f32(lo)) * (1.0 + np.cos(np.pi * ratio)))


def epoch_schedule(cfg, epoch):
    """(lr, ent_coef) of train_impl's epoch ``epoch`` (pufferlib.cu:1912-1948):
    cosine-annealed lr anchored at lr_anneal_from_epoch, times a linear warmup
    over lr_warmup_epochs counted from start_epoch; cosine-annealed entropy
    coefficient.  Both fp32 like the reference's.  With neither schedule on,
    the configured values come back unchanged."""
    lr, ent = cfg["learning_rate"], cfg["ent_coef"]
    total = max(1, int(cfg["total_epochs"]))
    if cfg["anneal_lr"] or cfg["lr_warmup_epochs"] > 0:
        lr = _f32(lr)
        if cfg["anneal_lr"]:
            lr_min = _f32(_f32(cfg["min_lr_ratio"]) * lr)
            t = max(0, epoch - int(cfg["lr_anneal_from_epoch"]))
            T = max(1, total - int(cfg["lr_anneal_from_epoch"]))
            lr = cosine_annealing(lr, lr_min, t, T)
        if cfg["lr_warmup_epochs"] > 0:
            ramp = epoch - int(cfg["start_epoch"])
            lr = _f32(lr * min(1.0, _f32(_f32(ramp + 1) / _f32(cfg["lr_warmup_epochs"]))))
    if cfg["anneal_ent_coef"]:
        ent_min = _f32(_f32(cfg["min_ent_coef_ratio"]) * _f32(ent))
        ent = cosine_annealing(ent, ent_min, epoch, total)
    return lr, ent


def _hypers(train):
    t = dict(TRAIN_DEFAULTS)
    t.update(train or {})
    return CPtcgHypers(t["learning_rate"], t["beta1"], t["beta2"], t["eps"],
                       t["max_grad_norm"], t["clip_coef"], t["vf_clip_coef"],
                       t["vf_coef"], t["ent_coef"], t["kl_skip_threshold"],
                       t["vf_skip_threshold"]), t


class PuffeRL:
    """Handle returned by :func:`create_pufferl` (owns a PtcgTrainer)."""

    def __init__(self, dm, train, seed=0):
        import torch
        if not torch.cuda.is_available():
            raise RuntimeError("CUDA is not available")
        self._torch = torch
        self.dims = dm
        self._cdims = dm.as_ctypes()
        self._chyp, self.train_cfg = _hypers(train)
        self.minibatch = int(self.train_cfg["minibatch_size"])
        self.seed = seed
        h = c_void_p()
        check(lib().ptcg_trainer_create(ctypes.byref(self._cdims), ctypes.byref(self._chyp),
                                        self.minibatch, ctypes.byref(h)))
        self._h = h
        self.packed_floats = lib().ptcg_packed_floats(ctypes.byref(self._cdims))
        self.obs_size = lib().ptcg_obs_size(ctypes.byref(self._cdims))
        self.rollout = None
        self.epoch = 0

    # -------------------------------------------------- weights
    def set_weights(self, packed):
        packed = np.ascontiguousarray(packed, dtype=np.float32).ravel()
        if packed.size != self.packed_floats:
            raise RuntimeError(f"Weight blob size mismatch: expected {self.packed_floats} floats, "
                               f"got {packed.size}")
        check(lib().ptcg_trainer_set_weights(self._h, fptr(packed)))

    def get_weights(self):
        out = np.empty(self.packed_floats, np.float32)
        check(lib().ptcg_trainer_get_weights(self._h, fptr(out)))
        return out

    def get_grads(self):
        out = np.empty(self.packed_floats, np.float32)
        check(lib().ptcg_trainer_get_grads(self._h, fptr(out)))
        return out

    def get_moments(self):
        m = np.empty(self.packed_floats, np.float32)
        v = np.empty(self.packed_floats, np.float32)
        check(lib().ptcg_trainer_get_moments(self._h, fptr(m), fptr(v)))
        return m, v

    def set_static(self, st):
        """Upload the static card / attack / skill tables of a static-table
        model (pt_static_upload, ptcg_model2.cu:383-419); ``st`` holds the
        arrays of :func:`synth.make_static`'s layout."""
        f = {k: np.ascontiguousarray(st[k], dtype=np.float32)
             for k in ("card_static", "att_static", "card_text", "att_text", "skill_text")}
        i = {k: np.ascontiguousarray(st[k], dtype=np.int32) for k in ("card_attacks", "card_skills")}
        dm = self.dims
        want = dict(card_static=(dm.n_cards, 58), att_static=(dm.n_attacks, 15), card_text=(dm.n_cards, 128),
                    att_text=(dm.n_attacks, 64), skill_text=(dm.n_skills, 64), card_attacks=(dm.n_cards, 4),
                    card_skills=(dm.n_cards, 2))
        for k, shp in want.items():
            a = f.get(k, i.get(k))
            if a.shape != shp:
                raise RuntimeError(f"static table {k}: shape {a.shape}, expected {shp}")
        check(lib().ptcg_trainer_set_static(self._h, *[fptr(f[k]) for k in ("card_static", "att_static",
                                                                            "card_text", "att_text", "skill_text")],
                                            i["card_attacks"].ctypes.data, i["card_skills"].ctypes.data))
        self._static = (f, i)   # keep the host copies alive for the call's duration

    def rollout_step(self, obs, n, seed, step, idx=None, stream=None, buf=0):
        """Forward ``n`` device obs rows with inference activations (rollout
        policy ``buf``: its own activations, so policies may run on different
        streams at once) and sample one action per row; returns device tensors
        (actions, logprobs, values)."""
        t = self._torch
        acts = t.empty(n, dtype=t.float32, device="cuda")
        lps, vals = t.empty_like(acts), t.empty_like(acts)
        check(lib().ptcg_trainer_rollout_on(self._h, buf, obs.data_ptr(), idx.data_ptr() if idx is not None else None,
                                            n, seed, step, acts.data_ptr(), lps.data_ptr(), vals.data_ptr(), stream))
        return acts, lps, vals

    def capture_rollout(self, slot, obs, n, seed, step_dev, actions, logprobs, values, idx=None):
        """Capture slot `slot`: the rollout step over these device buffers,
        the draw's step read from the device uint64 counter step_dev and
        advanced by one per replay (sync-free mode)."""
        check(lib().ptcg_trainer_capture_rollout(self._h, slot, obs.data_ptr(),
                                                 idx.data_ptr() if idx is not None else None, n, seed,
                                                 step_dev.data_ptr(), actions.data_ptr(), logprobs.data_ptr(),
                                                 values.data_ptr()))

    def rollout_output(self):
        """Device pointer of the last rollout call's (n, n_opt+1) output."""
        p = c_void_p()
        check(lib().ptcg_trainer_rollout_output(self._h, ctypes.byref(p)))
        return p.value

    def replay_rollout(self, slot, stream=None):
        check(lib().ptcg_trainer_replay_rollout(self._h, slot, stream))

    def step_count(self):
        v = ctypes.c_int32()
        check(lib().ptcg_trainer_step_count(self._h, ctypes.byref(v)))
        return v.value

    def set_hypers(self, **kw):
        """New hyper-parameters.  learning_rate and ent_coef reach the step
        through device scalars (a captured step follows them); a change of
        any other one drops the captured step (capture again)."""
        self.train_cfg.update(kw)
        self._chyp, self.train_cfg = _hypers(self.train_cfg)
        check(lib().ptcg_trainer_set_hypers(self._h, ctypes.byref(self._chyp)))

    def write_schedule(self, lr, ent_coef):
        """This epoch's lr and entropy coefficient into the device scalars
        (train_impl's cudaMemcpy to lr_ptr / ppo_bufs.ent_coef,
        pufferlib.cu:1933,1947); the configured base values stay."""
        h, _ = _hypers(dict(self.train_cfg, learning_rate=lr, ent_coef=ent_coef))
        check(lib().ptcg_trainer_set_hypers(self._h, ctypes.byref(h)))

    def hyper_ptrs(self):
        """Device addresses of the lr (double) and ent_coef (float) scalars."""
        lr, ent = c_void_p(), c_void_p()
        check(lib().ptcg_trainer_hyper_ptrs(self._h, ctypes.byref(lr), ctypes.byref(ent)))
        return lr.value, ent.value

    # -------------------------------------------------- device helpers
    def to_device(self, a, dtype=np.float32):
        t = self._torch.from_numpy(np.ascontiguousarray(a, dtype=dtype))
        return t.to("cuda")

    def buffers(self):
        p = [c_void_p() for _ in range(4)]
        check(lib().ptcg_trainer_buffers(self._h, *[ctypes.byref(x) for x in p]))
        return [x.value for x in p]

    def sync(self):
        check(lib().ptcg_trainer_sync(self._h))

    def forward_backward(self, obs, idx, inp, stream=None):
        """One forward + PPO loss + backward on device tensors (no optimizer)."""
        check(lib().ptcg_trainer_forward_backward(
            self._h, obs.data_ptr(), idx.data_ptr() if idx is not None else None,
            inp["actions"].data_ptr(), inp["logprobs"].data_ptr(),
            inp["advantages"].data_ptr(), inp["returns"].data_ptr(),
            inp["values"].data_ptr(), stream))

    def step(self, obs, idx, inp, stream=None):
        """One full minibatch step on device tensors (with the optimizer)."""
        check(lib().ptcg_trainer_step(
            self._h, obs.data_ptr(), idx.data_ptr() if idx is not None else None,
            inp["actions"].data_ptr(), inp["logprobs"].data_ptr(),
            inp["advantages"].data_ptr(), inp["returns"].data_ptr(),
            inp["values"].data_ptr(), stream))

    def capture_step(self, obs, idx, inp):
        """Capture one step over these device buffers into a HIP graph
        (sync-free mode); rewrite the buffers' contents, then replay_step."""
        check(lib().ptcg_trainer_capture_step(
            self._h, obs.data_ptr(), idx.data_ptr() if idx is not None else None,
            inp["actions"].data_ptr(), inp["logprobs"].data_ptr(), inp["advantages"].data_ptr(),
            inp["returns"].data_ptr(), inp["values"].data_ptr()))

    def replay_step(self, stream=None):
        check(lib().ptcg_trainer_replay_step(self._h, stream))

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            lib().ptcg_trainer_free(self._h)
            self._h = c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def create_pufferl(args):
    """args: {"dims": PtcgDims | dict, "train": {...}, "seed": int,
    "init_weights": packed blob | None, "static": static tables (static-table
    models), "precision": "fp32" | "bf16" (GEMM products), "sync_free": bool
    (compact row count kept on the device: no host read-back per forward, so
    the step can be graph-captured), "skip_masked_options": bool (default True:
    the option scorer runs only legal options in steps and rollouts),
    "sampler": "inverse_cdf" (default, the reference's rollout draw) | "gumbel"
    (Gumbel-max from counter-based noise)}.  Unknown dims keys
    raise."""
    dm = args.get("dims", dims_mod.CORE)
    if isinstance(dm, dict):
        dm = dims_mod.PtcgDims(**dm)
    pl = PuffeRL(dm, args.get("train", {}), args.get("seed", 0))
    if args.get("static") is not None:
        pl.set_static(args["static"])
    prec = args.get("precision", "fp32")
    if prec not in ("fp32", "bf16"):
        raise ValueError(f"precision must be 'fp32' or 'bf16', got {prec!r}")
    check(lib().ptcg_trainer_set_precision(pl._h, 1 if prec == "bf16" else 0))
    if args.get("sync_free", False):
        check(lib().ptcg_trainer_set_sync_free(pl._h, 1))
    if not args.get("skip_masked_options", True):
        check(lib().ptcg_trainer_set_skip_masked_options(pl._h, 0))
    sampler = args.get("sampler", "inverse_cdf")
    if sampler not in ("inverse_cdf", "gumbel"):
        raise ValueError(f"sampler must be 'inverse_cdf' or 'gumbel', got {sampler!r}")
    check(lib().ptcg_trainer_set_sampler(pl._h, 1 if sampler == "gumbel" else 0))
    opt = pl.train_cfg["optimizer"]
    if opt not in ("adam", "muon"):
        raise ValueError(f"optimizer must be 'adam' or 'muon', got {opt!r}")
    if opt == "muon":
        check(lib().ptcg_trainer_set_optimizer(pl._h, 1, float(pl.train_cfg["muon_wd_1d"])))
    init = args.get("init_weights")
    if init is None:
        from .params import init_blob
        init = init_blob(dm, args.get("seed", 0))
    pl.set_weights(init)
    return pl


def set_rollout(pl, obs, actions, logprobs, advantages, returns, values):
    """Upload a rollout (rows = observations) to device memory."""
    n = obs.shape[0]
    if obs.shape[1] != pl.obs_size:
        raise RuntimeError(f"rollout obs width {obs.shape[1]} != obs size {pl.obs_size}")
    pl.rollout = dict(
        obs=pl.to_device(obs), actions=pl.to_device(actions), logprobs=pl.to_device(logprobs),
        advantages=pl.to_device(advantages), returns=pl.to_device(returns),
        values=pl.to_device(values), n=n)


def set_segment_rollout(pl, obs, actions, logprobs, rewards, dones, values, horizon, layout="BT"):
    """A rollout as the reference's trainer holds it after collection:
    total_agents segments of ``horizon`` steps.  layout "TB": arrays in
    collection order (horizon, total_agents, ...), moved to the train layout
    (total_agents, horizon, ...) on the device (ptcg_transpose_102,
    train_impl :1863-1883); "BT": already in the train layout (row b*T + t).
    Rewards are clamped to [-1, 1] and the importance ratios set to 1, as
    train_impl does before its minibatch loop (:1889-1895)."""
    torch = pl._torch
    L = lib()
    T = int(horizon)
    obs = np.ascontiguousarray(obs, dtype=np.float32)
    n = obs.size // pl.obs_size
    if obs.size != n * pl.obs_size or n % T:
        raise RuntimeError(f"segment rollout: {obs.size} obs floats are not whole segments of {T} rows")
    S = n // T
    if layout not in ("BT", "TB"):
        raise ValueError(f"layout must be 'BT' or 'TB', got {layout!r}")
    if S > L.ptcg_prio_replay_max_segments():
        raise RuntimeError(f"segment rollout: {S} segments exceed {L.ptcg_prio_replay_max_segments()}")
    dev = lambda a, dt=torch.float32: torch.empty(a, dtype=dt, device="cuda")

    def train_layout(a, width, clamp=0):
        a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
        if a.size != n * width:
            raise RuntimeError(f"segment rollout: array of {a.size} floats, expected {n * width}")
        src = torch.from_numpy(a).to("cuda")
        if layout == "BT" and not clamp:
            return src
        out = dev(n * width)
        if layout == "BT":   # a [1, n*width] -> [n*width, 1] transpose is the clamped copy
            check(L.ptcg_transpose_102(out.data_ptr(), src.data_ptr(), 1, n * width, 1, clamp, None))
        else:
            check(L.ptcg_transpose_102(out.data_ptr(), src.data_ptr(), T, S, width, clamp, None))
        return out

    r = dict(obs=train_layout(obs, pl.obs_size), actions=train_layout(actions, 1),
             logprobs=train_layout(logprobs, 1), rewards=train_layout(rewards, 1, clamp=1),
             dones=train_layout(dones, 1), values=train_layout(values, 1).clone(), ratio=dev(n),
             advantages=dev(n), returns=dev(n), probs=dev(S), cdf=dev(S), row_prio=dev(n),
             idx=dev(max(S, pl.minibatch // T), torch.int32), mb_prio=dev(max(S, pl.minibatch // T)),
             row_idx=dev(pl.minibatch, torch.int32),
             rng_offset=torch.zeros(1, dtype=torch.int64, device="cuda"), n=n, horizon=T, segments=S)
    check(L.ptcg_fill(r["ratio"].data_ptr(), n, 1.0, None))
    pl.rollout = r


def _train_segments(pl):
    """train_impl's minibatch loop (pufferlib.cu:1963-2160): per minibatch,
    the negamax advantage over the whole rollout, a prioritized draw of
    minibatch / horizon segments, one step on their rows with their
    importance weights, then the step's ratios and new values written back
    into the rollout at the drawn segments."""
    L = lib()
    r, cfg = pl.rollout, pl.train_cfg
    T, S, B = r["horizon"], r["segments"], pl.minibatch
    if B % T:
        raise RuntimeError(f"minibatch {B} is not a whole number of {T}-step segments")
    mb_segs = B // T
    total_mb = int(cfg["replay_ratio"] * S * T / B)
    alpha, b0 = float(cfg["prio_alpha"]), float(cfg["prio_beta0"])
    beta = b0 + (1.0 - b0) * alpha * pl.epoch / max(1, int(cfg["total_epochs"]))
    seat = pl.dims.seat_col()
    P = lambda k: r[k].data_ptr()
    _, _, ratio_buf, nv_buf = pl.buffers()
    pl.write_schedule(*epoch_schedule(cfg, pl.epoch))
    try:
        for _ in range(total_mb):
            check(L.ptcg_negamax_advantage(P("values"), P("rewards"), P("dones"), P("ratio"), P("obs"),
                                           pl.obs_size, seat, P("advantages"), P("returns"),
                                           cfg["gamma"], cfg["gae_lambda"], cfg["vtrace_rho_clip"],
                                           cfg["vtrace_c_clip"], S, T, None))
            check(L.ptcg_prio_replay(P("advantages"), S, T, alpha, mb_segs, S, beta, pl.seed & ((1 << 64) - 1),
                                     P("rng_offset"), P("probs"), P("cdf"), P("idx"), P("mb_prio"),
                                     P("row_idx"), P("row_prio"), None))
            check(L.ptcg_trainer_set_prio(pl._h, P("row_prio")))
            pl.step(r["obs"], r["row_idx"], r)
            check(L.ptcg_index_copy(P("ratio"), P("idx"), ratio_buf, mb_segs, T, S, None))
            check(L.ptcg_index_copy(P("values"), P("idx"), nv_buf, mb_segs, T, S, None))
    finally:
        check(L.ptcg_trainer_set_prio(pl._h, None))
    pl.epoch += 1
    return log(pl)


def train(pl, index_lists=None):
    """One PPO update over the stored rollout.  A segment rollout
    (:func:`set_segment_rollout`) runs the reference's prioritized minibatch
    loop; a row rollout (:func:`set_rollout`) runs update_epochs epochs, each
    a fresh seeded permutation cut into minibatches (at most
    minibatches_per_epoch of them), or the given index lists.  Returns the
    loss dictionary of :func:`log`."""
    if pl.rollout is None:
        raise RuntimeError("train: no rollout set (call set_rollout)")
    if "horizon" in pl.rollout:
        if index_lists is not None:
            raise RuntimeError("train: index lists apply to row rollouts, not segment rollouts")
        return _train_segments(pl)
    from .synth import minibatch_indices
    r = pl.rollout
    B = pl.minibatch
    pl.write_schedule(*epoch_schedule(pl.train_cfg, pl.epoch))
    if index_lists is None:
        ep = int(pl.train_cfg["update_epochs"])
        per = min(int(pl.train_cfg["minibatches_per_epoch"]), r["n"] // B)
        index_lists = minibatch_indices(r["n"], B, ep * per, pl.seed + pl.epoch, epochs=ep)
    for idx in index_lists:
        idx = np.asarray(idx, dtype=np.int32)
        if idx.size != B:
            raise RuntimeError(f"minibatch index list has {idx.size} rows, trainer minibatch is {B}")
        pl.step(r["obs"], pl.to_device(idx, np.int32), r)
    pl.epoch += 1
    return log(pl)


def debug_forward(pl, rows):
    rows = np.ascontiguousarray(rows, dtype=np.float32)
    n = rows.size // pl.obs_size if rows.ndim == 1 else rows.shape[0]
    if rows.size != pl.minibatch * pl.obs_size:
        raise RuntimeError(f"debug_forward: need exactly {pl.minibatch * pl.obs_size} floats "
                           f"(minibatch {pl.minibatch} x obs {pl.obs_size}), got {rows.size}")
    out = np.empty((n, pl.dims.n_opt + 1), np.float32)
    check(lib().ptcg_trainer_debug_forward(pl._h, fptr(rows), n, fptr(out)))
    return out


def save_weights(pl, path):
    check(lib().ptcg_trainer_save_weights(pl._h, str(path).encode()))


def load_weights(pl, path):
    check(lib().ptcg_trainer_load_weights(pl._h, str(path).encode()))


def save_state(pl, path):
    """Optimizer state: the reference's PTCGSTA1 file (weights + Muon
    momentum, global step, epoch) with the Muon optimizer, PTCGADM1 (weights,
    Adam moments, step count) with Adam."""
    check(lib().ptcg_trainer_set_counters(pl._h, int(getattr(pl, "global_step", 0)), int(pl.epoch)))
    check(lib().ptcg_trainer_save_state(pl._h, str(path).encode()))


def load_state(pl, path):
    check(lib().ptcg_trainer_load_state(pl._h, str(path).encode()))
    gs, ep = ctypes.c_int64(), ctypes.c_int64()
    check(lib().ptcg_trainer_get_counters(pl._h, ctypes.byref(gs), ctypes.byref(ep)))
    if pl.train_cfg["optimizer"] == "muon":
        pl.global_step, pl.epoch = gs.value, ep.value


def log(pl, reset=True):
    out = np.zeros(10, np.float32)
    check(lib().ptcg_trainer_losses(pl._h, fptr(out), 1 if reset else 0))
    cnt = max(float(out[7]), 1.0)
    d = {k: float(out[i]) / cnt for i, k in enumerate(LOSS_KEYS)}
    d["minibatches"] = int(out[7])
    d["guard_skipped"] = int(out[8])
    d["grad_norm"] = float(out[9])
    return d


def close(pl):
    pl.close()
