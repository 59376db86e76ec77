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
The rollout's device buffers are allocated and owned through the library's
C ABI (:mod:`devmem`), and every computation runs in libptcg_amd.so.
"""
import ctypes
import time

import numpy as np

from . import dims as dims_mod
from . import devmem
from .devmem import DeviceArray
from .native import lib, check, fptr, CPtcgHypers, CPtcgLog, c_void_p, c_i32_p

# the loss sums of _C.log()["loss"] (bindings.cu:60-66), in the trainer's order
LOSS_KEYS = ("policy", "value", "entropy", "total", "old_kl", "kl", "clipfrac")
# _C.log()["perf"] phases: the reference's PROF_NAMES (pufferlib.cu:51-57),
# then the four parts of train_forward (model forward, PPO loss, model
# backward, gate + optimizer)
PERF_NAMES = ("rollout", "eval_gpu", "eval_env", "train_misc", "train_forward",
              "train_model_forward", "train_loss", "train_backward", "train_optimizer")


def _ptr(x):
    """Device address of a DeviceArray (or any object with data_ptr()), an
    int address, or None."""
    if x is None:
        return None
    return x if isinstance(x, int) else x.data_ptr()


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
        if devmem.device_count() < 1:
            raise RuntimeError("no GPU device is available")
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
        self.global_step = 0     # agent steps trained (the reference's global_step)
        self._start_time = self._last_log_time = time.time()
        self._last_log_step = 0

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
        streams at once) and sample one action per row; returns device arrays
        (actions, logprobs, values)."""
        acts, lps, vals = DeviceArray(n), DeviceArray(n), DeviceArray(n)
        check(lib().ptcg_trainer_rollout_on(self._h, buf, _ptr(obs), _ptr(idx), n, seed, step, acts.data_ptr(),
                                            lps.data_ptr(), vals.data_ptr(), stream))
        return acts, lps, vals

    def capture_rollout(self, slot, obs, n, seed, step_dev, actions, logprobs, values, idx=None):
        """Capture slot `slot`: the rollout step over these device buffers,
        the draw's step read from the device uint64 counter step_dev and
        advanced by one per replay (sync-free mode)."""
        check(lib().ptcg_trainer_capture_rollout(self._h, slot, _ptr(obs), _ptr(idx), n, seed, _ptr(step_dev),
                                                 _ptr(actions), _ptr(logprobs), _ptr(values)))

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
        """Host array -> DeviceArray (synchronous upload)."""
        return DeviceArray.from_numpy(np.ascontiguousarray(a, dtype=dtype))

    def buffers(self):
        p = [c_void_p() for _ in range(4)]
        check(lib().ptcg_trainer_buffers(self._h, *[ctypes.byref(x) for x in p]))
        return [x.value for x in p]

    def sync(self):
        check(lib().ptcg_trainer_sync(self._h))

    @staticmethod
    def _inputs(inp):
        return [_ptr(inp[k]) for k in ("actions", "logprobs", "advantages", "returns", "values")]

    def forward_backward(self, obs, idx, inp, stream=None):
        """One forward + PPO loss + backward on device arrays (no optimizer)."""
        check(lib().ptcg_trainer_forward_backward(self._h, _ptr(obs), _ptr(idx), *self._inputs(inp), stream))

    def step(self, obs, idx, inp, stream=None):
        """One full minibatch step on device arrays (with the optimizer).
        ``idx`` is a device int32 array, an int device address, or None."""
        check(lib().ptcg_trainer_step(self._h, _ptr(obs), _ptr(idx), *self._inputs(inp), stream))

    def capture_step(self, obs, idx, inp):
        """Capture one step over these device buffers into a HIP graph
        (sync-free mode); rewrite the buffers' contents, then replay_step."""
        check(lib().ptcg_trainer_capture_step(self._h, _ptr(obs), _ptr(idx), *self._inputs(inp)))

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
    dev = lambda a, dt=np.float32: DeviceArray(a, dt)

    def train_layout(a, width, clamp=0):
        a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
        if a.size != n * width:
            raise RuntimeError(f"segment rollout: array of {a.size} floats, expected {n * width}")
        src = DeviceArray.from_numpy(a)
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
             idx=dev(max(S, pl.minibatch // T), np.int32), mb_prio=dev(max(S, pl.minibatch // T)),
             row_idx=dev(pl.minibatch, np.int32), rng_offset=dev(1, np.int64), n=n, horizon=T, segments=S)
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
    check(L.ptcg_trainer_perf_mark(pl._h, 0, None))
    pl.write_schedule(*epoch_schedule(cfg, pl.epoch))
    check(L.ptcg_trainer_perf_mark(pl._h, 1, None))
    try:
        for _ in range(total_mb):
            check(L.ptcg_trainer_perf_mark(pl._h, 2, None))
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
    check(L.ptcg_trainer_perf_commit(pl._h, total_mb))
    pl.epoch += 1
    pl.global_step += r["n"]
    return {}


def train(pl, index_lists=None):
    """One PPO update over the stored rollout.  A segment rollout
    (:func:`set_segment_rollout`) runs the reference's prioritized minibatch
    loop; a row rollout (:func:`set_rollout`) runs update_epochs epochs, each
    a fresh seeded permutation cut into minibatches (at most
    minibatches_per_epoch of them), or the given index lists.  Returns an
    empty dict, as the reference's ``_C.train`` (bindings.cu:184-192): the
    losses accumulate on the device until :func:`log` reads them."""
    if pl.rollout is None:
        raise RuntimeError("train: no rollout set (call set_rollout)")
    if "horizon" in pl.rollout:
        if index_lists is not None:
            raise RuntimeError("train: index lists apply to row rollouts, not segment rollouts")
        return _train_segments(pl)
    from .synth import minibatch_indices
    L = lib()
    r = pl.rollout
    B = pl.minibatch
    check(L.ptcg_trainer_perf_mark(pl._h, 0, None))
    pl.write_schedule(*epoch_schedule(pl.train_cfg, pl.epoch))
    if index_lists is None:
        ep = int(pl.train_cfg["update_epochs"])
        per = min(int(pl.train_cfg["minibatches_per_epoch"]), r["n"] // B)
        index_lists = minibatch_indices(r["n"], B, ep * per, pl.seed + pl.epoch, epochs=ep)
    lists = [np.asarray(ix, dtype=np.int32) for ix in index_lists]
    for ix in lists:
        if ix.size != B:
            raise RuntimeError(f"minibatch index list has {ix.size} rows, trainer minibatch is {B}")
    # every minibatch's indices in one upload; step i reads slice i
    d_idx = DeviceArray.from_numpy(np.concatenate(lists)) if lists else None
    check(L.ptcg_trainer_perf_mark(pl._h, 1, None))
    for i in range(len(lists)):
        check(L.ptcg_trainer_perf_mark(pl._h, 2, None))
        pl.step(r["obs"], d_idx.data_ptr() + i * B * 4, r)
    check(L.ptcg_trainer_perf_commit(pl._h, len(lists)))   # synchronous: the steps are done
    del d_idx
    pl.epoch += 1
    pl.global_step += r["n"]
    return {}


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


def _rss_gb():
    """Resident set size of this process in GiB (/proc/self/status VmRSS,
    as bindings.cu:104-113 reads it), 0 where unavailable."""
    try:
        with open("/proc/self/status") as f:
            for line in f:
                if line.startswith("VmRSS:"):
                    return float(line.split()[1]) / (1024.0 * 1024.0)
    except OSError:
        pass
    return 0.0


def log(pl, reset=True):
    """The reference's ``_C.log(pl)`` (bindings.cu:15-118): SPS and
    agent_steps over the agent steps trained since the last log, uptime,
    epoch, the APPLIED learning rate read back from the device scalar the
    optimizer reads, ``env`` (empty: the environment is not part of this
    path), ``loss`` (the means of policy / value / entropy / total / old_kl /
    kl / clipfrac over the minibatches since the last log, and the gate's
    kl_skipped / vf_skipped counters; empty when no minibatch ran), ``perf``
    (seconds per phase from HIP events, the reference's keys plus the step's
    four parts; ``train`` = train_misc + train_forward) and ``util`` (GPU
    busy percent from amdgpu's sysfs, device memory in use, host RSS).
    Beyond the reference's keys: ``minibatches``, ``grad_norm`` (last step's
    norm before the clip), ``gate`` and ``ent_coef``.  ``reset`` clears the
    loss sums, the skip counters and the phase times, as the reference's
    log does."""
    st = CPtcgLog()
    check(lib().ptcg_trainer_set_counters(pl._h, int(pl.global_step), int(pl.epoch)))
    check(lib().ptcg_trainer_log(pl._h, ctypes.byref(st), 1 if reset else 0))
    return log_dict(pl, st, time.time(), reset)


def log_dict(pl, st, now, reset=True):
    """:func:`log`'s dictionary from a filled PtcgLog ``st`` (host-only)."""
    dt = now - pl._last_log_time
    sps = int((pl.global_step - pl._last_log_step) / dt) if dt > 0 else 0
    if reset:
        pl._last_log_time, pl._last_log_step = now, pl.global_step
    out = {"SPS": sps, "agent_steps": int(pl.global_step), "uptime": now - pl._start_time,
           "epoch": int(pl.epoch), "lr": float(st.lr), "env": {}}
    loss = {}
    n = float(st.n)
    if n > 0:
        inv = np.float32(1.0) / np.float32(n)      # the reference scales by 1/n in fp32
        for i, k in enumerate(LOSS_KEYS):
            loss[k] = float(np.float32(st.loss[i]) * inv)
        loss["kl_skipped"] = float(st.kl_skipped)
        loss["vf_skipped"] = float(st.vf_skipped)
    out["loss"] = loss
    perf = {k: float(st.perf_s[i]) for i, k in enumerate(PERF_NAMES)}
    perf["train"] = perf["train_misc"] + perf["train_forward"]
    out["perf"] = perf
    tot = float(st.vram_total_gb)
    out["util"] = {"gpu_percent": float(st.gpu_percent),
                   "gpu_mem": 100.0 * float(st.vram_used_gb) / tot if tot > 0 else 0.0,
                   "vram_used_gb": float(st.vram_used_gb), "vram_total_gb": tot, "cpu_mem_gb": _rss_gb()}
    out["minibatches"] = int(n)
    out["grad_norm"] = float(st.grad_norm)
    out["gate"] = float(st.gate)
    out["ent_coef"] = float(st.ent_coef)
    return out


def close(pl):
    pl.close()
