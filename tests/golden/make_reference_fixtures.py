"""Write golden vectors from the reference's own torch model (build container only).

Run here, where the reference checkout is mounted read-only at
``/root/reference``:

    python tests/golden/make_reference_fixtures.py

It imports ``ptcg.rl.model.PTCGTransformer`` (ptcg/rl/model.py:93-341) and
``native/tools/native_weights.py`` (``param_order`` / ``blob_to_sd``,
native_weights.py:45-113) from that checkout and records what they compute, so
the oracle's layer wiring (concat orders, head inputs, oracle-token features,
aux heads) and the packed blob's tensor order are pinned by the reference
itself rather than by a restatement.  Nothing here travels to the GPU box:
the outputs are the ``reference_*.npz`` files beside this script.

What stands in for what:

* ``build_tables()`` needs the engine SDK (``cg.api``, ptcg/rl/cards.py:39-40)
  and ``load_text_tables()`` reads ``data/embed_pca.npz``.  Both only PROVIDE
  the static card / attack / skill tables, which reach the module as plain
  arrays (model.py:104-112).  They are replaced by the seeded synthetic tables
  of ``synth.make_static``; no reference arithmetic is replaced.  The
  fixture records the tables' seed and SHA-256 so the test side rebuilds
  identical arrays.
* Weights: a seeded blob, laid out by the reference's own ``param_order`` and
  loaded through its own ``blob_to_sd``.  Each tensor is drawn as
  ``mean + std * z`` with ``z`` one PCG64 standard-normal stream over the
  whole blob; LayerNorm gains sit near 1, everything else is random, so two
  swapped same-shape tensors change the outputs.  The per-tensor
  (mean, std) table is stored; the test regenerates the blob from it
  without using this repository's own order.
* Observation rows: ``synth.make_obs(..., rich=True)`` frozen-layout rows
  (out-of-range / negative ids, tools, decision and attack ids), stored as
  is.  Pointers target valid tokens, the case the torch model's
  prefix-sliced gather shares with the native full-length one
  (model.py:253-260).

Recorded per case:

* ``names`` / ``shapes``: the reference's ``param_order()`` list;
* ``forward_train`` outputs (model.py:326-341): logits (torch fills illegal
  options with -1e9), oracle_v, blind_v, hand_pred, prize_logits (B, L) with
  L = the batch's longest valid prefix; ``forward_eval`` value under
  ``critic="blind"`` (model.py:315-320);
* gradients of two fixed weighted sums of those outputs, per tensor: the
  L2 norm, four projections on seeded N(0, 1) directions, and the full
  gradient of tensors with at most 4096 elements.
  ``A`` = legal logits + oracle_v + blind_v + hand_pred + prize_logits;
  ``C`` = legal logits + oracle_v (the decoder-output part of the native
  backward, ptcg_model4.cu:66-95).
"""
import os
import sys
from dataclasses import replace

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF = "/root/reference"

sys.path.insert(0, os.path.dirname(HERE))
from refvec import table_sha, make_blob, projections, SMALL   # noqa: E402


def blob_stats(names, shapes):
    """(mean, std) per tensor from its reference name and shape."""
    mean, std = [], []
    for name, shape in zip(names, shapes):
        if len(shape) == 1 and name.endswith(".weight"):      # LayerNorm gains
            mean.append(1.0), std.append(0.2)
        elif name.endswith(".bias"):
            mean.append(0.0), std.append(0.1)
        elif name in ("readout", "critic_readout") or "emb" in name:
            mean.append(0.0), std.append(0.5)
        else:                                                 # Linear weights (out, in)
            mean.append(0.0), std.append(1.0 / np.sqrt(shape[1]))
    return np.array(mean, np.float32), np.array(std, np.float32)


def main():
    sys.path.insert(0, ROOT)
    import __graft_entry__
    __graft_entry__.load_package()
    from ptcg_amd import dims, synth

    sys.path.insert(0, REF)
    sys.path.insert(0, os.path.join(REF, "native", "tools"))
    import torch
    import ptcg.rl.model as rm
    import native_weights as nw

    cases = [
        # the reference's frozen model (native_weights.py:24)
        dict(tag="frozen", d=256, heads=8, ffn=512, layers=4, B=8, seed=101),
        # the benchmark trunk's head count and FFN width on the frozen layout
        dict(tag="h4ffn1024", d=256, heads=4, ffn=1024, layers=2, B=6, seed=202),
    ]
    for c in cases:
        dm = replace(dims.FROZEN, heads=c["heads"], ffn=c["ffn"], layers=c["layers"])
        st_seed = c["seed"] + 1
        st = synth.make_static(dm, st_seed)
        tabs = (st["card_static"], st["card_attacks"].astype(np.int64),
                st["card_skills"].astype(np.int64), st["att_static"])
        rm.build_tables = lambda: tabs
        rm.load_text_tables = lambda: (st["card_text"], st["att_text"], st["skill_text"])

        # the reference's blob layout constants for this trunk
        nw.D, nw.HEADS, nw.FFN, nw.LAYERS = c["d"], c["heads"], c["ffn"], c["layers"]
        order = nw.param_order()
        names = [n for n, _ in order]
        shapes = [tuple(s) for _, s in order]
        mean, std = blob_stats(names, shapes)
        blob = make_blob(shapes, mean, std, c["seed"])

        torch.manual_seed(0)
        model = rm.PTCGTransformer(d=c["d"], layers=c["layers"], heads=c["heads"], ffn=c["ffn"],
                                   critic="oracle")
        res = model.load_state_dict(nw.blob_to_sd(blob), strict=False)
        buffers = {"card_static", "card_attacks", "card_skills", "att_static",
                   "card_text", "att_text", "skill_text"}
        assert set(res.missing_keys) == buffers, res.missing_keys
        assert not res.unexpected_keys, res.unexpected_keys
        model.eval()

        obs = synth.make_obs(dm, c["B"], seed=c["seed"] + 2, rich=True)
        o = torch.from_numpy(obs)
        out = model.forward_train(o)
        L = int(out["prize_logits"].shape[1])
        m0, m1 = dm.offsets()["opt_mask"]
        legal = torch.from_numpy(obs[:, m0:m1] != 0)

        rng = np.random.Generator(np.random.PCG64(c["seed"] + 3))
        w = {k: torch.from_numpy(rng.standard_normal(tuple(out[k].shape)).astype(np.float32))
             for k in ("logits", "oracle_v", "blind_v", "hand_pred", "prize_logits")}
        logit_term = (torch.where(legal, out["logits"], torch.zeros_like(out["logits"])) * w["logits"]).sum()
        obj_c = logit_term + (out["oracle_v"] * w["oracle_v"]).sum()
        obj_a = obj_c + sum((out[k] * w[k]).sum() for k in ("blind_v", "hand_pred", "prize_logits"))

        params = dict(model.named_parameters())
        grads = {}
        for tag, obj in (("A", obj_a), ("C", obj_c)):
            model.zero_grad()
            obj.backward(retain_graph=True)
            norms, projs, small = [], [], {}
            for i, n in enumerate(names):
                g = params[n].grad
                g = np.zeros(shapes[i], np.float32) if g is None else g.detach().numpy().astype(np.float32)
                norms.append(float(np.linalg.norm(g.astype(np.float64))))
                projs.append(projections(g, c["seed"] + (17 if tag == "A" else 29), i))
                if g.size <= SMALL:
                    small[n] = g
            grads[tag] = (np.array(norms), np.array(projs), small)

        model.critic_mode = "blind"
        _, v_blind = model.forward_eval(o)

        fx = dict(
            names=np.array(names), shape_flat=np.concatenate([np.array(s, np.int64) for s in shapes]),
            shape_rank=np.array([len(s) for s in shapes], np.int64),
            blob_mean=mean, blob_std=std, blob_seed=np.int64(c["seed"]),
            dims=np.array([c["d"], c["heads"], c["ffn"], c["layers"]], np.int64),
            static_seed=np.int64(st_seed), static_sha=np.array(table_sha(st)),
            obs=obs, L=np.int64(L),
            logits=out["logits"].detach().numpy(), oracle_v=out["oracle_v"].detach().numpy(),
            blind_v=out["blind_v"].detach().numpy(), hand_pred=out["hand_pred"].detach().numpy(),
            prize_logits=out["prize_logits"].detach().numpy(),
            unseen_mask=out["unseen_mask"].numpy(), token_ids=out["token_ids"].numpy(),
            eval_blind_v=v_blind.detach().numpy(),
            **{f"w_{k}": v.numpy() for k, v in w.items()},
        )
        for tag, (norms, projs, small) in grads.items():
            fx[f"g{tag}_norm"] = norms
            fx[f"g{tag}_proj"] = projs
            fx[f"g{tag}_proj_seed"] = np.int64(c["seed"] + (17 if tag == "A" else 29))
            fx[f"g{tag}_small_names"] = np.array(sorted(small))
            for n in sorted(small):
                fx[f"g{tag}_small/{n}"] = small[n]
        path = os.path.join(HERE, f"reference_{c['tag']}.npz")
        np.savez_compressed(path, **fx)
        print(f"{path}: {len(names)} tensors, {blob.size} floats, B={c['B']}, L={L}, "
              f"{os.path.getsize(path) / 1024:.0f} KiB")


if __name__ == "__main__":
    main()
