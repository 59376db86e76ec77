"""Golden vectors written by the reference's own torch model (tests/golden/).

``tests/golden/make_reference_fixtures.py`` imports ``PTCGTransformer`` and
``native_weights`` from the reference checkout and stores, per case, the
reference's blob order, a seeded blob recipe, observation rows, the
``forward_train`` / ``forward_eval`` outputs and per-tensor gradient
summaries.  This module rebuilds the inputs from a fixture file alone (the
blob from its stored per-tensor (mean, std) recipe, never from this
repository's own tensor order) and compares gradients against the stored
summaries.  Shared by the CPU and the GPU tests and by the fixture script.
"""
import hashlib
import os
from dataclasses import dataclass, replace

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = ("frozen", "h4ffn1024")
N_PROJ = 4       # random projections stored per gradient tensor
SMALL = 4096     # gradients of tensors up to this size are stored whole


def table_sha(st):
    h = hashlib.sha256()
    for k in sorted(st):
        a = np.ascontiguousarray(st[k])
        h.update(k.encode())
        h.update(str(a.dtype).encode())
        h.update(a.tobytes())
    return h.hexdigest()


def make_blob(shapes, mean, std, seed):
    """tensor i = mean_i + std_i * z over one PCG64 standard-normal stream."""
    counts = [int(np.prod(s)) for s in shapes]
    z = np.random.Generator(np.random.PCG64(seed)).standard_normal(sum(counts), dtype=np.float32)
    return (np.repeat(mean, counts) + np.repeat(std, counts) * z).astype(np.float32)


def projections(g, seed, i):
    """N_PROJ projections of gradient tensor i on seeded N(0, 1) directions."""
    r = np.random.Generator(np.random.PCG64([seed, i])).standard_normal((N_PROJ, g.size), dtype=np.float32)
    return r.astype(np.float64) @ np.asarray(g, np.float64).ravel()


@dataclass
class Fixture:
    tag: str
    z: dict
    dm: object
    names: list
    shapes: list
    blob: np.ndarray
    static: dict
    obs: np.ndarray
    L: int

    def legal(self):
        m0, m1 = self.dm.offsets()["opt_mask"]
        return self.obs[:, m0:m1] != 0

    def grad_check(self, tag, grads, tol=1e-4):
        """Compare {name: gradient} with the stored summaries of loss ``tag``
        ('A' or 'C'): per tensor |d norm| and |d projection| <= tol * norm
        (a projection of an error e on a unit-variance direction has
        standard deviation ||e||), whole small tensors at relative L2 <= tol.
        Returns the list of failures (name, what, value)."""
        z = self.z
        norms, projs, seed = z[f"g{tag}_norm"], z[f"g{tag}_proj"], int(z[f"g{tag}_proj_seed"])
        small = set(z[f"g{tag}_small_names"].tolist())
        bad = []
        for i, n in enumerate(self.names):
            g = np.asarray(grads[n], np.float64)
            ref_n = float(norms[i])
            scale = max(ref_n, 1e-30)
            got_n = float(np.linalg.norm(g))
            if ref_n == 0.0:
                if got_n > 1e-6:
                    bad.append((n, "nonzero where the reference is 0", got_n))
                continue
            if abs(got_n - ref_n) > tol * scale:
                bad.append((n, "norm", abs(got_n - ref_n) / scale))
            dp = np.abs(projections(g, seed, i) - projs[i]).max()
            if dp > 4 * tol * scale:
                bad.append((n, "projection", dp / scale))
            if n in small:
                r = z[f"g{tag}_small/{n}"].astype(np.float64)
                e = np.linalg.norm(g.ravel() - r.ravel()) / scale
                if e > tol:
                    bad.append((n, "elements", e))
        return bad


def load(tag):
    from ptcg_amd import dims, synth
    z = dict(np.load(os.path.join(GOLDEN, f"reference_{tag}.npz"), allow_pickle=False))
    ranks = z["shape_rank"].tolist()
    flat = z["shape_flat"].tolist()
    shapes, p = [], 0
    for r in ranks:
        shapes.append(tuple(int(v) for v in flat[p:p + r]))
        p += r
    names = [str(n) for n in z["names"]]
    d, heads, ffn, layers = (int(v) for v in z["dims"])
    dm = replace(dims.FROZEN, d=d, heads=heads, ffn=ffn, layers=layers)
    blob = make_blob(shapes, z["blob_mean"], z["blob_std"], int(z["blob_seed"]))
    st = synth.make_static(dm, int(z["static_seed"]))
    if table_sha(st) != str(z["static_sha"]):
        raise AssertionError("synth.make_static no longer reproduces the fixture's static tables")
    return Fixture(tag, z, dm, names, shapes, blob, st, z["obs"], int(z["L"]))
