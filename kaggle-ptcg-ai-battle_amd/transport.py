"""Rollout transport: pinned host mirrors of the env-side arrays, their device
counterparts and one stream per env buffer (the reference's vecenv GPU mode,
native/src/vecenv.h:498-545 allocation, :300-372 per-step copies), over the
ptcg_transport_* C ABI.

The host arrays are numpy views of pinned memory owned by the library: the
env writes observations / rewards / terminals into them and reads actions;
they are invalid after ``close()``.  Per (buffer, step):
``step(trainer, buf, slot)`` replays the buffer's captured rollout graph on
its stream and brings the actions back (checked stream sync); after the env
step, ``upload(buf)`` queues the new observations, rewards and terminals on
the same stream, ahead of the buffer's next forward.  Buffer b's graph runs
on the trainer's rollout policy b (its own activations), so ``launch`` (the
replay and the actions' download, without waiting) of several buffers keeps
their forwards in flight together, and ``wait(buf)`` is the checked sync.
"""
import ctypes

import numpy as np

from .native import check, lib

OBS, ACTIONS, REWARDS, TERMINALS, MASK, LOGPROBS, VALUES = range(7)


def _view(ptr, shape, dtype):
    n = int(np.prod(shape))
    buf = (ctypes.c_byte * (n * np.dtype(dtype).itemsize)).from_address(ptr)
    return np.frombuffer(buf, dtype=dtype, count=n).reshape(shape)


class RolloutTransport:
    def __init__(self, total_agents, num_buffers, obs_floats, num_atns=1, mask_bytes=0):
        h = ctypes.c_void_p()
        check(lib().ptcg_transport_create(total_agents, num_buffers, obs_floats, num_atns, mask_bytes,
                                          ctypes.byref(h)))
        self._h = h
        self.total_agents, self.num_buffers = total_agents, num_buffers
        self.agents_per_buffer = lib().ptcg_transport_agents_per_buffer(h)
        host = lambda w: lib().ptcg_transport_host(h, w)
        self.observations = _view(host(OBS), (total_agents, obs_floats), np.float32)
        self.actions = _view(host(ACTIONS), (total_agents, num_atns), np.float32)
        self.rewards = _view(host(REWARDS), (total_agents,), np.float32)
        self.terminals = _view(host(TERMINALS), (total_agents,), np.float32)
        self.action_mask = _view(host(MASK), (total_agents, mask_bytes), np.uint8) if mask_bytes else None

    def device_ptr(self, which):
        """Device base address of an array (OBS, ACTIONS, ..., LOGPROBS, VALUES)."""
        return lib().ptcg_transport_device(self._h, which)

    def stream(self, buf):
        return lib().ptcg_transport_stream(self._h, buf)

    def slice(self, buf):
        return slice(buf * self.agents_per_buffer, (buf + 1) * self.agents_per_buffer)

    def upload(self, buf):
        check(lib().ptcg_transport_upload(self._h, buf))

    def download(self, buf):
        check(lib().ptcg_transport_download(self._h, buf))

    def capture_rollout(self, pl, buf, slot, seed, step_dev):
        """Capture the trainer's rollout step over buffer `buf`'s device slices
        into slot `slot` (sync-free mode); step_dev: device uint64 counter."""
        check(lib().ptcg_transport_capture_rollout(self._h, pl._h, buf, slot, seed, step_dev.data_ptr()))

    def step(self, pl, buf, slot):
        check(lib().ptcg_transport_step(self._h, pl._h, buf, slot))

    def launch(self, pl, buf, slot):
        check(lib().ptcg_transport_launch(self._h, pl._h, buf, slot))

    def wait(self, buf):
        check(lib().ptcg_transport_wait(self._h, buf))

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            lib().ptcg_transport_free(self._h)
            self._h = ctypes.c_void_p()
            self.observations = self.actions = self.rewards = self.terminals = self.action_mask = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
