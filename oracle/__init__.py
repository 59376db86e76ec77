"""CPU oracle for the PTCG token-transformer PPO step — TEST INFRASTRUCTURE ONLY.

A from-scratch PyTorch (CPU, fp32/fp64) restatement of the reference's
algorithm for the training step, used as the checker for the HIP path:

* ``oracle.layout``  — obs-row offsets and weight-blob order
  (ptcg/rl/buffers.py:212-230, native/tools/native_weights.py:45-113).
* ``oracle.model``   — the policy forward with the native model's semantics
  (ptcg/rl/model.py:70-341 restated; native deviations from
  native/model/ptcg_model*.cu listed in that module); backward by autograd.
* ``oracle.ppo``     — the native PPO clipped loss with its hand-written
  gradient (native/src/pufferlib.cu:949-1363).
* ``oracle.adam``    — global-norm clip (native/src/muon.cu:107-114, same
  formula as torch's clip_grad_norm_) + torch.optim.Adam semantics, gated.
* ``oracle.step``    — one minibatch step and the multi-minibatch update.
* ``oracle.sampler`` — Philox4x32-10 counter RNG, the inverse-CDF action draw
  (native/src/pufferlib.cu:584-718) and the Gumbel-max draw with a logarithm
  reproducible in fp32.
* ``oracle.replay``  — the rollout-side steps of train_impl (numpy):
  transposes, negamax V-trace / GAE advantage, prioritized segment replay,
  index_copy write-back and the minibatch loop (pufferlib.cu:1847-2160).
* ``oracle.muon``    — the reference's optimizer, Muon (native/src/muon.cu:
  209-297), with Newton-Schulz orthogonalisation.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker or the CPU baseline — never on
the product path.

Pinning status (how each function is checked; see tests/test_oracle_*.py and
tests/test_golden_reference.py): every function here is pinned against
closed forms, torch library routines (F.layer_norm,
F.scaled_dot_product_attention, torch.autograd, torch.optim.Adam,
clip_grad_norm_, scipy.signal.lfilter for GAE), brute force on tiny inputs,
published known-answer vectors (Philox) or the reference's own constants
(obs size 10944, blob 4 465 812 floats).  The model's wiring (concat orders,
pointer targets, head inputs, oracle-token features, aux heads) and the full
blob tensor order are pinned by golden vectors produced by the reference's
own torch model and native_weights.param_order (tests/golden/, written by
tests/golden/make_reference_fixtures.py in the build container).
"""
