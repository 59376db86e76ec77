"""MI355X-native PPO training step for the PTCG token-transformer policy.

Submodules: ``dims`` (runtime sizes, obs layout), ``params`` (blob/arena
layout, initial weights), ``synth`` (seeded synthetic inputs), ``native``
(ctypes binding of the HIP C-ABI library), ``trainer`` (host-side mirror of
the reference trainer's Python API).
"""
from . import dims, params, synth  # noqa: F401
