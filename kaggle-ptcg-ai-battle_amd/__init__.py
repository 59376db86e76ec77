"""MI355X-native PPO training step for the PTCG token-transformer policy.

Submodules: ``dims`` (runtime sizes, obs layout), ``params`` (blob/arena
layout, initial weights), ``synth`` (seeded synthetic inputs), ``native``
(ctypes binding of the HIP C-ABI library), ``trainer`` (host-side mirror of
the reference trainer's Python API), ``transport`` (pinned host <-> device
rollout transport, one stream per env buffer).
"""
from . import dims, params, synth  # noqa: F401
