/*
 * ptcg_amd.h — C ABI of the MI355X-native PTCG token-transformer PPO step.
 *
 * Plain C types only: device pointers are float* / int32_t* into HIP device
 * memory, streams are passed as void* (a hipStream_t; NULL = the null stream).
 * Every function returns 0 on success and a negative code on failure; the
 * message is available from ptcg_last_error() (the reference aborts or throws
 * std::runtime_error with the same conditions, see each citation).
 *
 * Reference interfaces replaced (paths relative to the reference repo):
 *   - Encoder vtable of the PTCG model plugin: native/src/models.cu:16-47,
 *     native/model/ptcg_model4.cu:236-284, installed by native/src/ocean.cu:5-18.
 *   - PPO loss: ppo_loss_fwd_bwd, native/src/pufferlib.cu:1368-1449.
 *   - optimizer slot: muon_step, native/src/muon.cu:209 (here: clip + Adam).
 *   - trainer entry points: create_pufferl / train / debug_forward /
 *     save_weights / load_weights / save_state / load_state,
 *     native/src/bindings.cu:184-367,581-757; train_impl pufferlib.cu:1847.
 */
#ifndef PTCG_AMD_H
#define PTCG_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PTCG_OK 0
#define PTCG_ERR_ARG (-1)      /* bad argument / shape mismatch            */
#define PTCG_ERR_HIP (-2)      /* HIP runtime error                         */
#define PTCG_ERR_IO (-3)       /* file open/read/write failure              */
#define PTCG_ERR_UNSUPPORTED (-4)

/* Runtime sizes (the reference's compile-time PT_* macros,
 * ptcg_model.cu:14-87, and the obs layout of ptcg/rl/buffers.py:29-55).
 * tables: 0 = learned card/attack tables, 1 = static-table chain.
 * critic: 0 = blind value head, 1 = oracle critic.                         */
typedef struct PtcgDims {
    int l_tok, tok_int, tok_f, n_opt, opt_int, opt_f, global_f, dec_int, dec_f, oracle_f;
    int d, heads, ffn, layers, d_c, d_a, g;
    int n_cards, n_attacks, n_skills, n_zones, n_owners, n_opt_types, n_select_types, n_contexts;
    int tables, critic;
} PtcgDims;

/* Hyper-parameters of one minibatch step (the keys of the reference's
 * build_args train dict, native/train_native.py:251-280, plus Adam's).     */
typedef struct PtcgHypers {
    double lr, beta1, beta2, eps;         /* Adam (double: torch's scalars)    */
    float max_grad_norm;                  /* global-norm clip (muon.cu:216)    */
    float clip_coef, vf_clip_coef, vf_coef, ent_coef;   /* PPO              */
    float kl_skip_threshold, vf_skip_threshold;  /* gate; <= 0 disables     */
} PtcgHypers;

typedef struct PtcgModel PtcgModel;
typedef struct PtcgTrainer PtcgTrainer;

const char* ptcg_last_error(void);
int ptcg_abi_version(void);

/* ---- device memory (the trainer owns memory like the reference's
 * Allocator / alloc_create, native/src/kernels.cu:412-474; these give a
 * host driver its rollout buffers without another GPU runtime) ----------
 * alloc: zero-filled device bytes (bytes = 0 gives NULL).  memcpy dir: 0
 * host -> device, 1 device -> host (both synchronous: they wait for
 * `stream` first and return with the bytes in place), 2 device -> device
 * (ordered on `stream`).                                                   */
int ptcg_device_count(int* n);
int ptcg_device_alloc(int64_t bytes, void** out);
int ptcg_device_free(void* p);
int ptcg_memcpy(void* dst, const void* src, int64_t bytes, int dir, void* stream);
int ptcg_device_synchronize(void);
/* timing events (a hipEvent_t behind void*): elapsed_ms waits for b      */
int ptcg_event_create(void** ev);
int ptcg_event_record(void* ev, void* stream);
int ptcg_event_elapsed_ms(void* a, void* b, float* ms);
int ptcg_event_destroy(void* ev);

/* ---- layout (ptcg/rl/buffers.py:212-230; native_weights.py:45-113;
 *      kernels.cu:433-466 16 B alignment; pufferlib.cu:2366-2390) -------- */
int ptcg_obs_size(const PtcgDims* dims);
int ptcg_num_params(const PtcgDims* dims);
/* i-th tensor of the canonical blob order: name, rows, cols (0 for 1-D).   */
int ptcg_param_info(const PtcgDims* dims, int i, const char** name, int64_t* rows, int64_t* cols);
int64_t ptcg_packed_floats(const PtcgDims* dims);
int64_t ptcg_arena_floats(const PtcgDims* dims);
int ptcg_packed_to_arena(const PtcgDims* dims, const float* packed, float* arena);   /* host */
int ptcg_arena_to_packed(const PtcgDims* dims, const float* arena, float* packed);   /* host */

/* ---- model: the Encoder vtable, per entry point ----------------------- */
/* create_weights (ptcg_model4.cu:238-241)                                  */
int ptcg_model_create(const PtcgDims* dims, PtcgModel** out);
/* reg_params + alloc_create (ptcg_model4.cu:243-250): bind caller-owned
 * params / grads arenas, each ptcg_arena_floats() floats, 16 B aligned.    */
int ptcg_model_bind(PtcgModel* m, float* params_arena, float* grads_arena);
/* reg_train (ptcg_model4.cu:260-263): size activations for exactly n rows. */
int ptcg_model_reg_train(PtcgModel* m, int n);
/* reg_rollout (ptcg_model4.cu:265-267): inference activations for exactly
 * n rows — one block's buffers reused by every layer, no backward; the
 * training-only heads (blind value and belief heads of the oracle-critic
 * model) are skipped.  ptcg_model_backward then fails.                    */
int ptcg_model_reg_rollout(PtcgModel* m, int n);
/* forward (ptcg_model4.cu:269-275): obs rows -> *out (n, n_opt+1) =
 * [raw option scores || value], aliasing an internal buffer.
 * row_idx: optional int32 device array of n row indices into obs (NULL =
 * rows 0..n-1), replacing the trainer's minibatch copy (pufferlib.cu:2005). */
int ptcg_model_forward(PtcgModel* m, const float* obs, const int32_t* row_idx, int n,
                       float** out, void* stream);
/* Stage dumps for parity bisection (the reference's PTCG_DUMP_DIR,
 * ptcg_model3.cu:222-231,371-400, read by native/tools/stage_parity.py):
 * every named stage of the last forward as raw fp32 <dir>/<name>.bin —
 * card_vec, att_tab, tok_cat, tokp (N, l_tok, .), dec_in, g_out, d_out,
 * bc_out, keep, x0 (and x1..x_layers after a training forward), h
 * (N, l_seq, .), q_in, q_vec, sc_in (N, n_opt, .), out — rows the compact
 * trunk or the masked-option skip did not compute written as 0.  Set
 * PTCG_DUMP_DIR and every forward that is not being captured dumps at its
 * end.  Debug only: synchronous.                                          */
int ptcg_model_dump_stages(PtcgModel* m, const char* dir, void* stream);
/* backward (ptcg_model4.cu:277-281): grad (n, n_opt+1) = [d scores || d value];
 * OVERWRITES the grads arena (ptcg_model4.cu:15-21).                       */
int ptcg_model_backward(PtcgModel* m, const float* grad, void* stream);
/* free_weights + free_activations (ptcg_model4.cu:283-284).                */
void ptcg_model_free(PtcgModel* m);
/* pt_static_upload (ptcg_model2.cu:383-419), static-table models
 * (dims.tables == 1) only: host arrays card_static (n_cards, 58),
 * att_static (n_attacks, 15), card_text (n_cards, 128), att_text
 * (n_attacks, 64), skill_text (n_skills, 64), card_attacks (n_cards, 4) ids
 * in [0, n_attacks), card_skills (n_cards, 2) ids in [0, n_skills); 0 = an
 * empty slot.  Copied to device memory the model owns; required before the
 * first forward.                                                          */
int ptcg_model_set_static(PtcgModel* m, const float* card_static, const float* att_static,
                          const float* card_text, const float* att_text, const float* skill_text,
                          const int32_t* card_attacks, const int32_t* card_skills);
/* Product precision (the reference's USE_BF16 switch, compile-time there):
 * 0 = fp32 (default), 1 = the GEMMs' and attention's products on bf16 MFMA
 * (operands rounded to bf16, fp32 accumulation).  LayerNorm, softmax, loss,
 * weights and optimizer state stay fp32 in both.                          */
int ptcg_model_set_precision(PtcgModel* m, int prec);
/* Compact-layout row count handling (blind-critic models, whose trunk runs
 * only READOUT, valid-token and pointer-target rows).  0 (default): the
 * forward reads the row count back to the host once and sizes every trunk
 * launch for it.  1: no host read-back — launches are sized for the full
 * N * l_seq rows and stop at the count on the device, so forward / backward
 * stay stream-ordered and can be captured in a HIP graph, as the
 * reference's are (pufferlib.cu:2019-2140).  Results are the same.        */
int ptcg_model_set_sync_free(PtcgModel* m, int on);
/* Masked-option skipping, for callers whose loss masks illegal options
 * (the PPO loss maps opt_mask == 0 to the constant logit -1e4,
 * pufferlib.cu:949-962, so such a slot's score never reaches the loss and
 * its gradient is exactly 0 whenever the row has a legal option).  1: the
 * option scorer runs only each row's legal options (all of them when none is
 * legal), forward and backward; masked slots of the output read 0.  0
 * (default): every slot is scored, as the reference's forward does.       */
int ptcg_model_set_skip_masked_options(PtcgModel* m, int on);
/* ptcg_bind_train_graph (ptcg_model2.cu:323-330), oracle-critic models
 * (dims.critic == 1): device array of per-row returns the blind-value aux
 * loss regresses to, indexed like the obs rows of the forward (through its
 * row_idx when one was given).  Read by ptcg_model_backward.              */
int ptcg_model_bind_returns(PtcgModel* m, const float* returns);

/* ---- PPO loss fwd+bwd (pufferlib.cu:1368-1449; kernels :949-1363) -------
 * ent_coef is a device float read by the kernel, as the reference's is
 * (pufferlib.cu:199,1063: "by-value args get baked into the cuda graph").
 * dec_out (n, A+1) fused [scores || value]; mask (n rows at mask_stride,
 * 0 = illegal -> logit -1e4); per-row inputs gathered through row_idx when
 * non-NULL.  Writes grad (n, A+1) = [grad_logits || grad_value], ratio (n),
 * newvalue (n) (either may be NULL), stats[8] = 7 loss statistics + count
 * ADDED into (pufferlib.cu:1254-1284), and guard[2] = this minibatch's
 * (approx_kl, v_loss) when non-NULL.  All pointers are device pointers.    */
int ptcg_ppo_loss_fwd_bwd(const float* dec_out, int n, int A,
                          const float* mask, int64_t mask_stride, const int32_t* row_idx,
                          const float* actions, const float* old_logprobs,
                          const float* advantages, const float* returns,
                          const float* values, const float* prio,
                          float clip_coef, float vf_clip_coef, float vf_coef, const float* ent_coef,
                          float* grad, float* ratio, float* newvalue,
                          float* stats, float* guard, void* stream);

/* ---- the PPO loss without allocation.  No counterpart in the reference:
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and results as ptcg_ppo_loss_fwd_bwd, which allocates its
 * per-block partials on first use; this one keeps them in a static device
 * array of the library (one per GPU, held until the process ends) and calls
 * no allocator.  n <= PT_PPO_NOALLOC_MAX_ROWS, else PTCG_ERR_ARG.  All calls
 * on one GPU share the array: calls that overlap on one GPU race.          */
#define PT_PPO_NOALLOC_MAX_ROWS 65536
int ptcg_ppo_loss_fwd_bwd_noalloc(const float* dec_out, int n, int A,
                                  const float* mask, int64_t mask_stride, const int32_t* row_idx,
                                  const float* actions, const float* old_logprobs,
                                  const float* advantages, const float* returns,
                                  const float* values, const float* prio,
                                  float clip_coef, float vf_clip_coef, float vf_coef, const float* ent_coef,
                                  float* grad, float* ratio, float* newvalue,
                                  float* stats, float* guard, void* stream);

/* ---- gate (kl_gate_kernel, pufferlib.cu:1292-1302): gate[0] = 1 apply /
 * 0 skip, from guard[0..1] = (approx_kl, v_loss).  skipped: null or two
 * adjacent device floats, the reference's KL_GUARD_SKIPPED and
 * KL_GUARD_SKIPPED_VF (pufferlib.cu:37-38): skipped[0] += 1 - gate (every
 * veto), skipped[1] += 1 when the value test failed.                      */
int ptcg_kl_gate(const float* guard, float kl_threshold, float vf_threshold,
                 float* gate, float* skipped, void* stream);

/* ---- optimizer slot (muon_step, muon.cu:209-297 -> clip + Adam) ---------
 * One fused pass over the flat arenas (n floats, n % 4 == 0, 16 B aligned):
 * g' = g * min(max_norm / (||g||_2 + 1e-6), 1); Adam moments m, v; weights
 * updated with bias correction for step t = *step + 1 (torch.optim.Adam
 * semantics).  lr: device double read by the kernel (the reference's
 * lr_ptr, muon.cu:92-100), so a captured step follows the host's writes.
 * step: device int32 count of applied steps, advanced on the device.  gate: optional device float; when it reads 0 the call changes
 * nothing (weights, m, v, step untouched).  norm_out: optional device float
 * receiving ||g||_2 before clipping.  workspace: device buffer of
 * ptcg_adam_workspace_floats() floats.  grads are read, not modified.      */
int64_t ptcg_adam_workspace_floats(void);
int ptcg_adam_step(float* weights, float* grads, float* m, float* v, int64_t n,
                   const double* lr, double beta1, double beta2, double eps, float max_grad_norm,
                   const float* gate, int32_t* step, float* norm_out, float* workspace,
                   void* stream);
/* The same step with the learning rate read from a device float: the type
 * of the reference trainer's own lr_ptr (muon.cu:96-99, written by
 * train_impl at pufferlib.cu:1933), so that a reference-side caller binds
 * its lr_ptr directly.  The float is widened to double before Adam's
 * scalar arithmetic; everything else is ptcg_adam_step.                   */
int ptcg_adam_step_lrf(float* weights, float* grads, float* m, float* v, int64_t n,
                       const float* lr, double beta1, double beta2, double eps, float max_grad_norm,
                       const float* gate, int32_t* step, float* norm_out, float* workspace,
                       void* stream);

/* ---- Muon, the reference's optimizer (muon.cu:154-297) ------------------
 * muon_init + muon_post_create: momentum arena (zeroed) and Newton-Schulz
 * workspaces for the tensor shapes of dims; lr is kept on the device
 * (the reference's lr_ptr).  momentum = the trainer's beta1 (pufferlib.cu:
 * 2660), weight_decay applies to >= 2-D tensors (the reference passes 0),
 * wd_1d to 1-D tensors (muon_wd_1d).                                       */
typedef struct PtcgMuon PtcgMuon;
int ptcg_muon_create(const PtcgDims* dims, double lr, double momentum, double weight_decay, double wd_1d,
                     PtcgMuon** out);
void ptcg_muon_free(PtcgMuon* m);
/* the host's learning-rate write (train_impl's cudaMemcpy to lr_ptr, pufferlib.cu:1937); synchronous */
int ptcg_muon_set_lr(PtcgMuon* m, float lr);
/* device pointer of the momentum arena (ptcg_arena_floats(dims) floats, params layout) */
float* ptcg_muon_momentum(PtcgMuon* m);
/* muon_step (muon.cu:215-297) on the params / grads arenas: global-norm clip
 * (coefficient min(max_grad_norm / (||g|| + 1e-6), 1)), then per tensor
 * Nesterov momentum + 5 Newton-Schulz iterations + scaled update (>= 2-D) or
 * EMA momentum + update (1-D).  grads are read, not modified (the reference
 * clips and transforms them in place).  gate: optional device float, 0 = the
 * call changes neither weights nor momentum.  grad_norm_out: optional device
 * float receiving ||g||_2 before clipping.                                 */
int ptcg_muon_step(PtcgMuon* m, float* weights, const float* grads, float max_grad_norm, const float* gate,
                   float* grad_norm_out, void* stream);

/* ---- action sampler (sample_logits, pufferlib.cu:584-718) ---------------
 * One discrete head of A options per row of dec_out (n, A+1) = [scores ||
 * value]: masked (mask == 0 -> -1e4, rows at mask_stride, gathered through
 * row_idx when non-NULL) softmax, inverse-CDF draw with
 * u = Philox4x32-10(counter = (row, step), key = seed) in (0, 1) where the
 * reference advances a per-row cuRAND state.  Writes actions (option index
 * as float), logprobs, values (last column; may be NULL) and, when
 * non-NULL, the uniforms used.                                            */
int ptcg_sample_actions(const float* dec_out, int n, int A, const float* mask, int64_t mask_stride,
                        const int32_t* row_idx, uint64_t seed, uint64_t step, float* actions,
                        float* logprobs, float* values, float* uniforms, void* stream);

/* ---- Gumbel-max sampler.  No counterpart in the reference (its rollout
 * draws by inverse CDF, above); for callers that need draws reproducible
 * bit for bit from (seed, step, row, option) or from given noise.
 * action = argmax_j (l_j + g_j), ties to the lowest j, over the same safe,
 * masked logits (mask == 0 -> -1e4); g_j = -log(-log u_j) with
 * u_j = Philox4x32-10(counter = (row, step lo, step hi, 1 + j/4), key = seed),
 * word j % 4, mapped to (0, 1) as above, and log evaluated by a fixed
 * sequence of correctly rounded fp32 operations (so a CPU restatement
 * reproduces every g_j).  noise: optional device (n, A) array of g_j to use
 * instead (NULL = generate).  logprobs = l_a - logsumexp(l) (fp32), values
 * = the last column.  noise_out: optional (n, A), the g_j used.  A <= 64.  */
int ptcg_sample_actions_gumbel(const float* dec_out, int n, int A, const float* mask, int64_t mask_stride,
                               const int32_t* row_idx, const float* noise, uint64_t seed, uint64_t step,
                               float* actions, float* logprobs, float* values, float* noise_out, void* stream);

/* ---- rollout-side steps of train_impl (pufferlib.cu:1847-2160) ----------
 * All buffers are device fp32 (int32 where named) on the caller's stream.
 *
 * transpose_102 (kernels.cu:179-188; train_impl :1863-1883): dst[b, a, c] =
 * src[a, b, c] for shapes [A, B, C] -> [B, A, C]; clamp != 0 also clamps to
 * [-1, 1] on the way (the rewards' clamp_precision_kernel, :1889-1891).   */
int ptcg_transpose_102(float* dst, const float* src, int A, int B, int C, int clamp, void* stream);
/* fill_precision_kernel (:1893-1895; the importance ratios' reset to 1).  */
int ptcg_fill(float* dst, int64_t n, float value, void* stream);
/* negamax V-trace/GAE, ptcg_puff_advantage / k_negamax_adv
 * (ptcg_model2.cu:287-321, after the advantages' puf_zero at :1966): rows
 * of T steps in (B, T) layout; seat_t = obs[(b*T + t)*obs_stride + seat_col]
 * (the actor-seat global feature); advantages[:, T-1] = 0.  returns
 * (optional) = values + advantages, which select_copy forms (:1773).      */
int ptcg_negamax_advantage(const float* values, const float* rewards, const float* dones,
                           const float* importance, const float* obs, int64_t obs_stride, int seat_col,
                           float* advantages, float* returns, float gamma, float lambda, float rho_clip,
                           float c_clip, int B, int T, void* stream);
/* prioritized replay, prio_replay_cuda (:1455-1591): per segment
 * p_b = (sum_t |adv_bt|)^alpha (non-finite -> 0), probs = (p + 1e-6) /
 * (sum p + 1e-6) (written to probs, B floats), cdf = inclusive scan (B
 * floats); n_samples draws with replacement u_k = Philox4x32-10(counter =
 * (offset + k, 0, 1), key = seed) where the reference draws cuRAND
 * Philox(seed, offset + k); idx_k = first b with cdf_b >= u_k (B-1 if none);
 * mb_prio_k = (total_agents * probs[idx_k])^-anneal_beta; *rng_offset (device
 * int64) += n_samples.  Optional outputs for a step that reads rows through
 * row_idx: row_idx (n_samples * T int32) = idx_k * T + t; row_prio (B * T
 * floats, rollout rows) gets mb_prio_k at the sampled segments' rows.
 * B <= ptcg_prio_replay_max_segments().                                    */
int ptcg_prio_replay_max_segments(void);
int ptcg_prio_replay(const float* advantages, int B, int T, float prio_alpha, int n_samples,
                     int total_agents, float anneal_beta, uint64_t seed, int64_t* rng_offset,
                     float* probs, float* cdf, int32_t* idx, float* mb_prio, int32_t* row_idx,
                     float* row_prio, void* stream);
/* index_copy (:1747-1754; the ratio / new-value write-back :2146-2160):
 * dst row idx[i] <- src row i, rows of row_floats floats; rows whose index
 * is outside [0, dst_rows) are skipped.                                   */
int ptcg_index_copy(float* dst, const int32_t* idx, const float* src, int n_idx, int row_floats,
                    int dst_rows, void* stream);

/* ---- trainer (create_pufferl / train / debug_forward / weights IO) ----- */
int ptcg_trainer_create(const PtcgDims* dims, const PtcgHypers* hyp, int minibatch,
                        PtcgTrainer** out);
void ptcg_trainer_free(PtcgTrainer* t);
/* New hyper-parameters.  lr and ent_coef go to device scalars read by the
 * step's kernels (train_impl's per-call cudaMemcpy to lr_ptr and
 * ppo_bufs.ent_coef, pufferlib.cu:1912-1948), so a captured step follows
 * them.  A change of any other field drops the captured step (it is a launch
 * argument there); replay_step then fails until capture_step runs again.   */
int ptcg_trainer_set_hypers(PtcgTrainer* t, const PtcgHypers* hyp);
/* Device addresses of those two scalars (a double and a float), for callers
 * that write the schedule on a stream of their own.                      */
int ptcg_trainer_hyper_ptrs(PtcgTrainer* t, double** lr, float** ent_coef);
/* packed blob <-> live arena (bindings.cu:202-215,339-367), host buffers   */
int ptcg_trainer_set_weights(PtcgTrainer* t, const float* packed);
int ptcg_trainer_get_weights(PtcgTrainer* t, float* packed);
int ptcg_trainer_get_grads(PtcgTrainer* t, float* packed);
int ptcg_trainer_get_moments(PtcgTrainer* t, float* m_packed, float* v_packed);
int ptcg_trainer_load_weights(PtcgTrainer* t, const char* path);
int ptcg_trainer_save_weights(PtcgTrainer* t, const char* path);
/* full state: "PTCGADM1" header (step count, n) + weights + m + v, packed.  */
int ptcg_trainer_save_state(PtcgTrainer* t, const char* path);
int ptcg_trainer_load_state(PtcgTrainer* t, const char* path);
/* debug_forward (bindings.cu:221-250): host obs (minibatch rows) -> host
 * out (minibatch, n_opt+1); synchronous.                                  */
int ptcg_trainer_debug_forward(PtcgTrainer* t, const float* obs_host, int n, float* out_host);
/* Rollout step of the policy (net_callback_wrapper -> policy_forward ->
 * sample_logits, pufferlib.cu:757-946): forward n obs rows (device, through
 * row_idx when non-NULL) with inference activations on the trainer's
 * current weights, then sample one action per row (ptcg_sample_actions,
 * mask = the rows' opt_mask section).  actions, logprobs, values: device
 * arrays of n floats.                                                     */
int ptcg_trainer_rollout(PtcgTrainer* t, const float* obs, const int32_t* row_idx, int n,
                         uint64_t seed, uint64_t step, float* actions, float* logprobs,
                         float* values, void* stream);
/* The same on rollout policy `buf` (0 <= buf < 64): each policy has its own
 * inference activations (registered for the n of its calls), so calls on
 * different policies may run concurrently on different streams — the
 * reference's per-buffer rollout threads and streams (pufferlib.cu:502-509,
 * vecenv.h:259-384).  ptcg_trainer_rollout is policy 0.                   */
int ptcg_trainer_rollout_on(PtcgTrainer* t, int buf, const float* obs, const int32_t* row_idx, int n,
                            uint64_t seed, uint64_t step, float* actions, float* logprobs,
                            float* values, void* stream);
/* Optimizer of the trainer's steps: 0 = clip + Adam (default), 1 = Muon
 * (ptcg_muon_*, momentum = hyp.beta1, weight decay 0 on >= 2-D tensors,
 * wd_1d on 1-D tensors, lr = hyp.lr).  save_state / load_state then use the
 * reference's PTCGSTA1 format (bindings.cu:257-337: header, packed weights,
 * packed momentum) instead of PTCGADM1.                                    */
int ptcg_trainer_set_optimizer(PtcgTrainer* t, int kind, double wd_1d);
/* global_step / epoch carried in PTCGSTA1 headers (bindings.cu:257-262)    */
int ptcg_trainer_set_counters(PtcgTrainer* t, int64_t global_step, int64_t epoch);
int ptcg_trainer_get_counters(PtcgTrainer* t, int64_t* global_step, int64_t* epoch);
/* Graph capture of the rollout step (the reference's per-(t, buf) rollout
 * graphs, pufferlib.cu:757-946): capture_rollout records, into slot `slot`,
 * ptcg_trainer_rollout over these device buffers with the draw's step read
 * from the device counter *step_dev (uint64) and advanced by one at the end
 * of every replay; replay_rollout launches slot `slot` on `stream`.  Sync-free
 * mode; every slot uses the same row count n.                              */
int ptcg_trainer_capture_rollout(PtcgTrainer* t, int slot, const float* obs, const int32_t* row_idx, int n,
                                 uint64_t seed, uint64_t* step_dev, float* actions, float* logprobs,
                                 float* values);
int ptcg_trainer_replay_rollout(PtcgTrainer* t, int slot, void* stream);
/* capture_rollout on rollout policy `buf` (see ptcg_trainer_rollout_on):
 * slots captured on different policies may replay concurrently.           */
int ptcg_trainer_capture_rollout_on(PtcgTrainer* t, int buf, int slot, const float* obs, const int32_t* row_idx,
                                    int n, uint64_t seed, uint64_t* step_dev, float* actions, float* logprobs,
                                    float* values);
/* The rollout's draw (ptcg_trainer_rollout, capture_rollout): 0 = inverse
 * CDF (default, the reference's sample_logits), 1 = Gumbel-max
 * (ptcg_sample_actions_gumbel).  A change drops captured rollout slots.   */
int ptcg_trainer_set_sampler(PtcgTrainer* t, int kind);
/* device pointer of the rollout policy's (roll_n, n_opt+1) output of the
 * last rollout call (for tests)                                           */
int ptcg_trainer_rollout_output(PtcgTrainer* t, float** dec_out);
/* floats per observation row of the trainer's dims (ptcg_obs_size).       */
int ptcg_trainer_obs_size(PtcgTrainer* t);

/* ---- rollout transport (vecenv.h GPU mode) ------------------------------
 * Pinned host mirrors of the env-side arrays, their device counterparts and
 * one stream per env buffer: the reference's cudaHostAlloc(Portable) /
 * cudaMalloc pairs and per-buffer streams (native/src/vecenv.h:498-545).
 * total_agents split into num_buffers contiguous slices of
 * agents_per_buffer agents; per agent: obs_floats observation floats,
 * num_atns action floats, one reward, one terminal, mask_bytes of action
 * mask (0: none; this model reads its mask from the observation row), and
 * on the device only one log-prob and one value (the rollout buffers).    */
typedef struct PtcgTransport PtcgTransport;
enum PtcgTransportArray { PTCG_TR_OBS = 0, PTCG_TR_ACTIONS = 1, PTCG_TR_REWARDS = 2, PTCG_TR_TERMINALS = 3,
                          PTCG_TR_MASK = 4, PTCG_TR_LOGPROBS = 5, PTCG_TR_VALUES = 6, PTCG_TR_COUNT = 7 };
int ptcg_transport_create(int total_agents, int num_buffers, int64_t obs_floats, int num_atns, int mask_bytes,
                          PtcgTransport** out);
int ptcg_transport_free(PtcgTransport* x);
/* base pointers of an array (host: NULL for log-probs and values)         */
void* ptcg_transport_host(PtcgTransport* x, int which);
void* ptcg_transport_device(PtcgTransport* x, int which);
/* the buffer's stream (hipStream_t)                                       */
void* ptcg_transport_stream(PtcgTransport* x, int buf);
int ptcg_transport_agents_per_buffer(PtcgTransport* x);
/* async H2D of the buffer's observations, rewards, terminals and mask on
 * its stream (vecenv.h:355-372, after the env step)                       */
int ptcg_transport_upload(PtcgTransport* x, int buf);
/* D2H of the buffer's actions on its stream, then a checked stream sync
 * (vecenv.h:311-337: the env must not step on stale actions)              */
int ptcg_transport_download(PtcgTransport* x, int buf);
/* ptcg_trainer_capture_rollout_on(t, buf, slot, ...) over the buffer's
 * device slices (observations in, actions / log-probs / values out;
 * num_atns 1): buffer b runs on rollout policy b, so buffers' steps may
 * overlap                                                                 */
int ptcg_transport_capture_rollout(PtcgTransport* x, PtcgTrainer* t, int buf, int slot, uint64_t seed,
                                   uint64_t* step_dev);
/* one rollout step of a buffer (net_callback + the actions' trip,
 * vecenv.h:309-337): replay slot `slot` on the buffer's stream, then
 * ptcg_transport_download                                                 */
int ptcg_transport_step(PtcgTransport* x, PtcgTrainer* t, int buf, int slot);
/* the same split in two, so that one host thread can keep several buffers'
 * forwards in flight: launch = replay + async D2H of the actions (returns at
 * once); wait = the buffer's checked stream sync                          */
int ptcg_transport_launch(PtcgTransport* x, PtcgTrainer* t, int buf, int slot);
int ptcg_transport_wait(PtcgTransport* x, int buf);

/* ptcg_model_set_precision on the trainer's models (train and rollout).  */
int ptcg_trainer_set_precision(PtcgTrainer* t, int prec);
/* ptcg_model_set_sync_free on the trainer's models (train and rollout).   */
int ptcg_trainer_set_sync_free(PtcgTrainer* t, int on);
/* Masked-option skipping in the trainer's own steps and rollouts (default
 * on: its PPO loss and sampler mask those slots); debug_forward always
 * scores every slot.                                                      */
int ptcg_trainer_set_skip_masked_options(PtcgTrainer* t, int on);
/* ptcg_model_set_static on the trainer's model.                          */
int ptcg_trainer_set_static(PtcgTrainer* t, const float* card_static, const float* att_static,
                            const float* card_text, const float* att_text, const float* skill_text,
                            const int32_t* card_attacks, const int32_t* card_skills);
/* One PPO minibatch step on device data (the body of train_impl's loop,
 * pufferlib.cu:2039-2105): forward -> loss fwd+bwd -> backward -> gate ->
 * clip + Adam.  obs rows and the per-row inputs (actions, old log-probs,
 * advantages, returns, old values) are read through row_idx (device int32,
 * minibatch entries; NULL = rows 0..minibatch-1).  The action mask is the
 * obs row's opt_mask section.                                              */
int ptcg_trainer_step(PtcgTrainer* t, const float* obs, const int32_t* row_idx,
                      const float* actions, const float* old_logprobs,
                      const float* advantages, const float* returns, const float* values,
                      void* stream);
/* Importance weights of the policy loss (the reference's mb_prio, read per
 * row as g.prio, pufferlib.cu:1040): a device array read through row_idx
 * like the other per-row inputs (e.g. ptcg_prio_replay's row_prio), used by
 * every later step until replaced; NULL = weight 1 (the default).          */
int ptcg_trainer_set_prio(PtcgTrainer* t, const float* prio);
/* Graph capture of the training step (the reference's captured train
 * graph, pufferlib.cu:2019-2140): capture_step records one
 * ptcg_trainer_step over the given device buffers into a HIP graph (sync-free
 * mode only: every node is a kernel; nothing runs during capture);
 * replay_step launches it on `stream`.  The buffers' addresses are baked
 * in: write each minibatch's indices / inputs into the same buffers before
 * a replay.  Re-capturing replaces the graph.  set_optimizer, set_precision,
 * set_sync_free, set_skip_masked_options, a new prio pointer and a change of
 * a by-value hyper-parameter (set_hypers) drop it.                          */
int ptcg_trainer_capture_step(PtcgTrainer* t, const float* obs, const int32_t* row_idx,
                              const float* actions, const float* old_logprobs,
                              const float* advantages, const float* returns, const float* values);
int ptcg_trainer_replay_step(PtcgTrainer* t, void* stream);
/* The same step without the optimizer (grads left in the grads arena).    */
int ptcg_trainer_forward_backward(PtcgTrainer* t, const float* obs, const int32_t* row_idx,
                                  const float* actions, const float* old_logprobs,
                                  const float* advantages, const float* returns,
                                  const float* values, void* stream);
/* ---- log (_C.log, bindings.cu:15-118) ----------------------------------
 * Phases of PtcgLog.perf_s: the reference's PROF_NAMES (pufferlib.cu:43-57)
 * in its order, then this build's split of train_forward into the step's
 * four parts.                                                             */
#define PTCG_PERF_ROLLOUT 0
#define PTCG_PERF_EVAL_GPU 1
#define PTCG_PERF_EVAL_ENV 2
#define PTCG_PERF_TRAIN_MISC 3
#define PTCG_PERF_TRAIN_FORWARD 4
#define PTCG_PERF_FORWARD 5      /* model forward                          */
#define PTCG_PERF_LOSS 6         /* PPO loss fwd + bwd                     */
#define PTCG_PERF_BACKWARD 7     /* model backward                         */
#define PTCG_PERF_OPTIMIZER 8    /* gate + clip + Adam (or Muon)           */
#define PTCG_PERF_N 9
typedef struct PtcgLog {
    /* sums since the last reset (losses_puf, pufferlib.cu:1254-1284):
     * policy, value, entropy, total, old_kl, kl, clipfrac                  */
    float loss[7];
    float n;               /* minibatches in those sums (LOSS_N)            */
    float kl_skipped;      /* gate vetoes since the last reset              */
    float vf_skipped;      /* ... of which the value test failed           */
    float gate;            /* the gate's last decision (kept over resets)   */
    float grad_norm;       /* last step's global grad norm before the clip  */
    float lr;              /* the APPLIED lr, read back from the device     */
    float ent_coef;        /* the applied entropy coefficient (device)      */
    float gpu_percent;     /* amdgpu gpu_busy_percent of this device, or -1 */
    float pad_;
    double perf_s[PTCG_PERF_N];   /* seconds per phase since the last reset */
    double vram_used_gb, vram_total_gb;   /* hipMemGetInfo                 */
    int64_t global_step, epoch;          /* ptcg_trainer_set_counters       */
} PtcgLog;
/* Synchronous.  reset != 0 zeroes the loss sums, the two skip counters and
 * perf_s afterwards (the reference zeroes losses, SKIPPED / SKIPPED_VF and
 * its profile; the gate keeps its value).                                  */
int ptcg_trainer_log(PtcgTrainer* t, PtcgLog* out, int reset);
/* Phase timing (the reference's profile.events, pufferlib.cu:1851-2185).
 * mark 0 / 1: start / end of train's pre-loop setup; mark 2: start of a
 * minibatch's misc work (advantage, replay draw, index upload).  An eager
 * ptcg_trainer_step on a stream that is not capturing records the end of
 * the misc work and the ends of its forward, loss, backward and optimizer.
 * perf_commit (synchronous) adds the pre-loop span once and the last
 * minibatch's spans times `minibatches` (the reference's accounting,
 * pufferlib.cu:2174-2185); spans whose marks were not recorded add 0.      */
int ptcg_trainer_perf_mark(PtcgTrainer* t, int mark, void* stream);
int ptcg_trainer_perf_commit(PtcgTrainer* t, int minibatches);
/* host seconds spent outside the trainer's streams (rollouts, eval), added
 * to phase `phase` as the reference adds its rollout wall time
 * (bindings.cu:170-177)                                                    */
int ptcg_trainer_perf_add(PtcgTrainer* t, int phase, double seconds);
/* device pointer of the last forward's (minibatch, n_opt+1) output and of
 * the PPO grad buffer (for tests).                                         */
int ptcg_trainer_buffers(PtcgTrainer* t, float** dec_out, float** ppo_grad,
                         float** ratio, float** newvalue);
int ptcg_trainer_sync(PtcgTrainer* t);
/* number of applied optimizer steps (device counter), synchronous          */
int ptcg_trainer_step_count(PtcgTrainer* t, int32_t* out);

#ifdef __cplusplus
}
#endif
#endif /* PTCG_AMD_H */
