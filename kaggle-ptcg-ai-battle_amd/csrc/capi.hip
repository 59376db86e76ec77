// extern "C" surface: errors, layout, PPO / gate / Adam entry points and the
// trainer (include/ptcg_amd.h documents each entry point and the reference
// interface it replaces).
#include "model.h"

#include <ctype.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <deque>
#include <mutex>
#include <string>
#include <vector>

// ------------------------------------------------------------ errors
static thread_local char g_err[1024] = "";

void ptcg_set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

extern "C" const char* ptcg_last_error(void) { return g_err; }
extern "C" int ptcg_abi_version(void) { return 1; }

// ------------------------------------------------------------ layout
ObsOff pt_obs_offsets(const PtcgDims& d) {
    // ptcg/rl/buffers.py:212-227: sections back to back in this order
    ObsOff o;
    int cur = 0;
    o.tok_int = cur; cur += d.l_tok * d.tok_int;
    o.tok_float = cur; cur += d.l_tok * d.tok_f;
    o.opt_int = cur; cur += d.n_opt * d.opt_int;
    o.opt_float = cur; cur += d.n_opt * d.opt_f;
    o.opt_mask = cur; cur += d.n_opt;
    o.global_f = cur; cur += d.global_f;
    o.dec_int = cur; cur += d.dec_int;
    o.dec_float = cur; cur += d.dec_f;
    o.oracle = cur; cur += d.oracle_f;
    o.size = cur;
    return o;
}

DimsX pt_dims_x(const PtcgDims& d) {
    DimsX x;
    x.l_seq = d.l_tok + 1;
    x.dh = d.d / d.heads;
    x.tok_in = 2 * d.d_c + d.tok_f + PT_ZONE_E + PT_OWNER_E;
    x.dec_in = PT_SEL_E + PT_CTX_E + 2 * d.d_c + 2 * d.d_a + 2 * d.d_c + d.dec_f;
    x.bcast_in = d.g + PT_DEC_H;
    x.q_in = PT_TYPE_E + 2 * d.d + 2 * PT_OPT_E + d.opt_f;
    x.score_in = 3 * d.d + d.g + PT_DEC_H;
    x.val_in = d.d + d.g;
    x.card_in = PT_ID_C + PT_CARD_STATIC + PT_CARD_TEXT + 2 * d.d_a + 2 * d.d_c;
    x.att_in = PT_ID_A + PT_ATT_STATIC + PT_ATT_TEXT;
    x.sk_in = PT_ID_A + PT_SKILL_TEXT;
    x.orc_in = d.d_c + 6;
    x.n_orc = PT_N_HAND + PT_N_SPLIT + PT_N_PRIZE;
    x.l_crit = 1 + x.l_seq + x.n_orc;
    return x;
}

static const char* intern(const std::string& s) {
    static std::mutex mu;
    static std::deque<std::string> pool;
    std::lock_guard<std::mutex> lk(mu);
    for (auto& p : pool)
        if (p == s) return p.c_str();
    pool.push_back(s);
    return pool.back().c_str();
}

// Canonical blob order: native/tools/native_weights.py:34-92 (PT_PARAMS,
// ptcg_model.cu:95-126); learned tables replace the 13 static-chain tensors
// with card_table / attack_table; the blind critic drops the oracle critic
// and aux tensors.
int pt_param_table(const PtcgDims& d, ParamDef* out, int cap) {
    std::vector<ParamDef> v;
    auto add = [&](const std::string& n, long r, long c) { v.push_back({intern(n), r, c}); };
    const DimsX x = pt_dims_x(d);
    const long D = d.d, DC = d.d_c, DA = d.d_a, G = d.g;
    if (d.tables == 1) {
        add("card_id_emb.weight", d.n_cards, PT_ID_C);
        add("attack_id_emb.weight", d.n_attacks, PT_ID_A);
        add("skill_id_emb.weight", d.n_skills, PT_ID_A);
        add("attack_mlp.0.weight", DA, x.att_in); add("attack_mlp.0.bias", DA, 0);
        add("skill_mlp.0.weight", DC, x.sk_in); add("skill_mlp.0.bias", DC, 0);
        add("card_mlp.0.weight", x.card_in, 0); add("card_mlp.0.bias", x.card_in, 0);
        add("card_mlp.1.weight", PT_CARD_H, x.card_in); add("card_mlp.1.bias", PT_CARD_H, 0);
        add("card_mlp.3.weight", DC, PT_CARD_H); add("card_mlp.3.bias", DC, 0);
    } else if (d.tables == 0) {
        add("card_table", d.n_cards, DC);
        add("attack_table", d.n_attacks, DA);
    } else {
        ptcg_set_error("param table: unknown tables mode %d", d.tables);
        return PTCG_ERR_ARG;
    }
    add("zone_emb.weight", d.n_zones, PT_ZONE_E);
    add("owner_emb.weight", d.n_owners, PT_OWNER_E);
    add("token_proj.weight", D, x.tok_in); add("token_proj.bias", D, 0);
    add("readout", D, 0);
    add("global_mlp.0.weight", G, d.global_f); add("global_mlp.0.bias", G, 0);
    add("global_mlp.2.weight", G, G); add("global_mlp.2.bias", G, 0);
    add("sel_type_emb.weight", d.n_select_types, PT_SEL_E);
    add("ctx_emb.weight", d.n_contexts, PT_CTX_E);
    add("dec_mlp.0.weight", PT_DEC_H, x.dec_in); add("dec_mlp.0.bias", PT_DEC_H, 0);
    add("dec_mlp.2.weight", PT_DEC_H, PT_DEC_H); add("dec_mlp.2.bias", PT_DEC_H, 0);
    add("bcast.weight", D, x.bcast_in); add("bcast.bias", D, 0);
    auto block = [&](const std::string& p) {
        add(p + ".ln1.weight", D, 0); add(p + ".ln1.bias", D, 0);
        add(p + ".qkv.weight", 3 * D, D); add(p + ".qkv.bias", 3 * D, 0);
        add(p + ".proj.weight", D, D); add(p + ".proj.bias", D, 0);
        add(p + ".ln2.weight", D, 0); add(p + ".ln2.bias", D, 0);
        add(p + ".ffn.0.weight", d.ffn, D); add(p + ".ffn.0.bias", d.ffn, 0);
        add(p + ".ffn.2.weight", D, d.ffn); add(p + ".ffn.2.bias", D, 0);
    };
    for (int i = 0; i < d.layers; ++i) block("blocks." + std::to_string(i));
    add("ln_f.weight", D, 0); add("ln_f.bias", D, 0);
    add("opt_type_emb.weight", d.n_opt_types, PT_TYPE_E);
    add("opt_card.weight", PT_OPT_E, DC); add("opt_card.bias", PT_OPT_E, 0);
    add("opt_attack.weight", PT_OPT_E, DA); add("opt_attack.bias", PT_OPT_E, 0);
    add("q_mlp.0.weight", D, x.q_in); add("q_mlp.0.bias", D, 0);
    add("q_mlp.2.weight", D, D); add("q_mlp.2.bias", D, 0);
    add("score_mlp.0.weight", PT_SC_H, x.score_in); add("score_mlp.0.bias", PT_SC_H, 0);
    add("score_mlp.2.weight", 1, PT_SC_H); add("score_mlp.2.bias", 1, 0);
    add("value_mlp.0.weight", PT_VAL_H, x.val_in); add("value_mlp.0.bias", PT_VAL_H, 0);
    add("value_mlp.2.weight", 1, PT_VAL_H); add("value_mlp.2.bias", 1, 0);
    if (d.critic == 1) {
        add("oracle_proj.weight", D, x.orc_in); add("oracle_proj.bias", D, 0);
        add("critic_readout", D, 0);
        block("critic_blocks.0");
        add("oracle_value_mlp.0.weight", PT_VAL_H, x.val_in); add("oracle_value_mlp.0.bias", PT_VAL_H, 0);
        add("oracle_value_mlp.2.weight", 1, PT_VAL_H); add("oracle_value_mlp.2.bias", 1, 0);
        add("aux_hand.weight", d.n_cards, x.val_in); add("aux_hand.bias", d.n_cards, 0);
        add("aux_prize.weight", 1, D); add("aux_prize.bias", 1, 0);
    }
    if ((int)v.size() > cap) {
        ptcg_set_error("param table: %zu entries exceed capacity %d", v.size(), cap);
        return PTCG_ERR_ARG;
    }
    for (size_t i = 0; i < v.size(); ++i) out[i] = v[i];
    return (int)v.size();
}

static int table(const PtcgDims* dims, std::vector<ParamDef>& v) {
    PT_REQUIRE(dims != nullptr, "null dims");
    v.resize(256);
    int n = pt_param_table(*dims, v.data(), 256);
    if (n < 0) return n;
    v.resize(n);
    return PTCG_OK;
}

static inline long numel(const ParamDef& p) { return p.rows * (p.cols > 0 ? p.cols : 1); }

extern "C" int ptcg_obs_size(const PtcgDims* dims) {
    PT_REQUIRE(dims != nullptr, "null dims");
    return pt_obs_offsets(*dims).size;
}

extern "C" int ptcg_num_params(const PtcgDims* dims) {
    std::vector<ParamDef> v;
    PT_TRY(table(dims, v));
    return (int)v.size();
}

extern "C" int ptcg_param_info(const PtcgDims* dims, int i, const char** name, int64_t* rows, int64_t* cols) {
    std::vector<ParamDef> v;
    PT_TRY(table(dims, v));
    PT_REQUIRE(i >= 0 && i < (int)v.size(), "param_info: index %d out of range", i);
    if (name) *name = v[i].name;
    if (rows) *rows = v[i].rows;
    if (cols) *cols = v[i].cols;
    return PTCG_OK;
}

extern "C" int64_t ptcg_packed_floats(const PtcgDims* dims) {
    std::vector<ParamDef> v;
    PT_TRY(table(dims, v));
    int64_t n = 0;
    for (auto& p : v) n += numel(p);
    return n;
}

// kernels.cu:433-466 — each tensor starts at a 16 B (4-float) boundary
extern "C" int64_t ptcg_arena_floats(const PtcgDims* dims) {
    std::vector<ParamDef> v;
    PT_TRY(table(dims, v));
    int64_t off = 0;
    for (auto& p : v) off = ((off + 3) & ~3L) + numel(p);
    return (off + 3) & ~3L;
}

// pufferlib.cu:2366-2390
static int packed_arena(const PtcgDims* dims, const float* src, float* dst, bool to_arena) {
    std::vector<ParamDef> v;
    PT_TRY(table(dims, v));
    PT_REQUIRE(src && dst, "packed/arena: null buffer");
    if (to_arena) memset(dst, 0, sizeof(float) * ptcg_arena_floats(dims));
    int64_t off = 0, poff = 0;
    for (auto& p : v) {
        off = (off + 3) & ~3L;
        const long ne = numel(p);
        if (to_arena) memcpy(dst + off, src + poff, ne * sizeof(float));
        else memcpy(dst + poff, src + off, ne * sizeof(float));
        off += ne;
        poff += ne;
    }
    return PTCG_OK;
}
extern "C" int ptcg_packed_to_arena(const PtcgDims* dims, const float* packed, float* arena) {
    return packed_arena(dims, packed, arena, true);
}
extern "C" int ptcg_arena_to_packed(const PtcgDims* dims, const float* arena, float* packed) {
    return packed_arena(dims, arena, packed, false);
}

// ------------------------------------------------------------ device memory
// The trainer owns its device memory as the reference's does (Allocator /
// alloc_create, kernels.cu:412-474); these let a host-side driver hold the
// rollout's device buffers and move bytes without another runtime.
extern "C" int ptcg_device_count(int* n) {
    PT_REQUIRE(n, "device_count: null argument");
    *n = 0;
    const hipError_t e = hipGetDeviceCount(n);
    if (e != hipSuccess) *n = 0;
    return PTCG_OK;
}

extern "C" int ptcg_device_alloc(int64_t bytes, void** out) {
    PT_REQUIRE(out && bytes >= 0, "device_alloc: bad arguments");
    *out = nullptr;
    if (bytes == 0) return PTCG_OK;
    PT_HIP(hipMalloc(out, (size_t)bytes));
    const hipError_t e = hipMemset(*out, 0, (size_t)bytes);
    if (e != hipSuccess) {
        (void)hipFree(*out);
        *out = nullptr;
        ptcg_set_error("device_alloc: hipMemset: %s", hipGetErrorString(e));
        return PTCG_ERR_HIP;
    }
    return PTCG_OK;
}

// waits for the device first: work launched on any stream may still read p
extern "C" int ptcg_device_free(void* p) {
    if (!p) return PTCG_OK;
    PT_HIP(hipDeviceSynchronize());
    PT_HIP(hipFree(p));
    return PTCG_OK;
}

// dir: 0 host -> device, 1 device -> host, 2 device -> device.  Host <->
// device copies are synchronous (they return with the bytes in place);
// device -> device is ordered on `stream`.
extern "C" int ptcg_memcpy(void* dst, const void* src, int64_t bytes, int dir, void* stream) {
    PT_REQUIRE(bytes >= 0 && dir >= 0 && dir <= 2, "memcpy: bad arguments (bytes %lld, dir %d)",
               (long long)bytes, dir);
    if (bytes == 0) return PTCG_OK;
    PT_REQUIRE(dst && src, "memcpy: null pointer");
    if (dir == 2) {
        PT_HIP(hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream));
        return PTCG_OK;
    }
    PT_HIP(hipStreamSynchronize((hipStream_t)stream));
    PT_HIP(hipMemcpy(dst, src, (size_t)bytes, dir == 0 ? hipMemcpyHostToDevice : hipMemcpyDeviceToHost));
    return PTCG_OK;
}

extern "C" int ptcg_device_synchronize(void) {
    PT_HIP(hipDeviceSynchronize());
    return PTCG_OK;
}

// timing events for host drivers (hipEvent_t behind void*)
extern "C" int ptcg_event_create(void** ev) {
    PT_REQUIRE(ev, "event_create: null argument");
    hipEvent_t e = nullptr;
    PT_HIP(hipEventCreate(&e));
    *ev = e;
    return PTCG_OK;
}

extern "C" int ptcg_event_record(void* ev, void* stream) {
    PT_REQUIRE(ev, "event_record: null event");
    PT_HIP(hipEventRecord((hipEvent_t)ev, (hipStream_t)stream));
    return PTCG_OK;
}

// milliseconds from a to b; waits for b
extern "C" int ptcg_event_elapsed_ms(void* a, void* b, float* ms) {
    PT_REQUIRE(a && b && ms, "event_elapsed_ms: null argument");
    PT_HIP(hipEventSynchronize((hipEvent_t)b));
    PT_HIP(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
    return PTCG_OK;
}

extern "C" int ptcg_event_destroy(void* ev) {
    if (ev) PT_HIP(hipEventDestroy((hipEvent_t)ev));
    return PTCG_OK;
}

// ------------------------------------------------------------ PPO / gate / Adam
extern "C" int ptcg_ppo_loss_fwd_bwd(const float* dec_out, int n, int A, const float* mask,
                                     int64_t mask_stride, const int32_t* row_idx, const float* actions,
                                     const float* old_logprobs, const float* advantages,
                                     const float* returns, const float* values, const float* prio,
                                     float clip_coef, float vf_clip_coef, float vf_coef, const float* ent_coef,
                                     float* grad, float* ratio, float* newvalue, float* stats,
                                     float* guard, void* stream) {
    PT_REQUIRE(dec_out && mask && actions && old_logprobs && advantages && returns && values && grad && ent_coef,
               "ppo_loss: null input");
    hipStream_t s = (hipStream_t)stream;
    // per-block partials live in a per-thread scratch sized for the largest n seen
    static thread_local float* part = nullptr;
    static thread_local long part_cap = 0;
    const long need = pt_ppo_partial_floats(n);
    if (need > part_cap) {
        if (part) PT_HIP(hipFree(part));
        part = nullptr;
        PT_HIP(hipMalloc(&part, need * sizeof(float)));
        part_cap = need;
    }
    return pt_ppo_loss(dec_out, n, A, mask, mask_stride, row_idx, actions, old_logprobs, advantages,
                       returns, values, prio, clip_coef, vf_clip_coef, vf_coef, ent_coef, grad,
                       ratio, newvalue, stats, guard, part, s);
}

// ---- the PPO loss without allocation, for callers that cannot allocate
// device memory (code under graph capture, serving loops, harnesses that
// forbid hipMalloc).  Its per-block partials live in `scratch`, a
// file-scope device array of PT_PPO_NOALLOC_MAX_ROWS rows' worth.  The
// kernels write every partial they later read, so nothing needs clearing.
// Each GPU has its own copy; all calls on one GPU share it, so calls that
// overlap on one GPU (other streams, other threads) race.
static __device__ __align__(256) float scratch[(PT_PPO_NOALLOC_MAX_ROWS / 16) * 7];   // 16 rows a partial

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};   // device address of `scratch`, per device
}  // namespace

// Device address of this device's `scratch`, looked up once per device with
// that device current (the array's host-side name is not a device address).
static int scratch_ptr(float** out) {
    int dev = -1;
    PT_HIP(hipGetDevice(&dev));
    PT_REQUIRE(dev >= 0 && dev < kMaxDevices, "ppo_loss_noalloc: device %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        PT_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        PT_REQUIRE(p != nullptr, "ppo_loss_noalloc: no device address for the scratch array");
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_ptr[dev];
    return PTCG_OK;
}

extern "C" int ptcg_ppo_loss_fwd_bwd_noalloc(const float* dec_out, int n, int A, const float* mask,
                                             int64_t mask_stride, const int32_t* row_idx, const float* actions,
                                             const float* old_logprobs, const float* advantages,
                                             const float* returns, const float* values, const float* prio,
                                             float clip_coef, float vf_clip_coef, float vf_coef,
                                             const float* ent_coef, float* grad, float* ratio, float* newvalue,
                                             float* stats, float* guard, void* stream) {
    PT_REQUIRE(dec_out && mask && actions && old_logprobs && advantages && returns && values && grad && ent_coef,
               "ppo_loss_noalloc: null input");
    PT_REQUIRE(n >= 2 && n <= PT_PPO_NOALLOC_MAX_ROWS,
               "ppo_loss_noalloc: n=%d rows outside [2, %d] (the scratch array's limit)", n,
               PT_PPO_NOALLOC_MAX_ROWS);
    PT_REQUIRE(pt_ppo_partial_floats(n) <= (long)(sizeof(scratch) / sizeof(float)),
               "ppo_loss_noalloc: %ld partials exceed the scratch array", pt_ppo_partial_floats(n));
    float* part = nullptr;
    PT_TRY(scratch_ptr(&part));
    return pt_ppo_loss(dec_out, n, A, mask, mask_stride, row_idx, actions, old_logprobs, advantages, returns,
                       values, prio, clip_coef, vf_clip_coef, vf_coef, ent_coef, grad, ratio, newvalue, stats,
                       guard, part, (hipStream_t)stream);
}

extern "C" int ptcg_kl_gate(const float* guard, float kl_threshold, float vf_threshold, float* gate,
                            float* skipped, void* stream) {
    PT_REQUIRE(guard && gate, "kl_gate: null buffer");
    return pt_kl_gate(guard, kl_threshold, vf_threshold, gate, skipped, (hipStream_t)stream);
}

extern "C" int ptcg_adam_step(float* weights, float* grads, float* m, float* v, int64_t n, const double* lr,
                              double beta1, double beta2, double eps, float max_grad_norm,
                              const float* gate, int32_t* step, float* norm_out, float* workspace,
                              void* stream) {
    PT_REQUIRE(weights && grads && m && v && lr && step && workspace, "adam_step: null buffer");
    return pt_adam_step(weights, grads, m, v, n, lr, beta1, beta2, eps, max_grad_norm, gate, step,
                        norm_out, workspace, (hipStream_t)stream);
}

extern "C" int ptcg_adam_step_lrf(float* weights, float* grads, float* m, float* v, int64_t n, const float* lr,
                                  double beta1, double beta2, double eps, float max_grad_norm,
                                  const float* gate, int32_t* step, float* norm_out, float* workspace,
                                  void* stream) {
    PT_REQUIRE(weights && grads && m && v && lr && step && workspace, "adam_step_lrf: null buffer");
    return pt_adam_step(weights, grads, m, v, n, lr, beta1, beta2, eps, max_grad_norm, gate, step,
                        norm_out, workspace, (hipStream_t)stream);
}

extern "C" int64_t ptcg_adam_workspace_floats(void) { return pt_adam_ws_floats(); }

// ------------------------------------------------------------ trainer
long pt_model_arena(const PtcgModel* m);
// phase marks: 0 / 1 pre-loop start / end, 2 misc start, 3 step start (misc
// end), 4 forward end, 5 loss end, 6 backward end, 7 optimizer end
constexpr int PT_NMARK = 8;
// trainer stats floats: [0..6] loss sums, [7] minibatches, [8] / [9] the
// gate's two skip counters (adjacent, as the reference's), [10] grad norm
constexpr int PT_ST_SKIP = 8, PT_ST_NORM = 10, PT_ST_FLOATS = 11;
float* pt_model_out(const PtcgModel* m);

struct PtcgTrainer {
    PtcgDims dm;
    PtcgHypers hyp;
    ObsOff off;
    int B = 0;
    long arena = 0, packed = 0;
    PtcgModel* model = nullptr;
    char* mem = nullptr;
    float *P, *Gr, *M, *V;
    float *grad, *ratio, *newvalue, *stats, *guard, *gate, *ppo_part, *adam_ws, *dbg_obs;
    int32_t* step;
    // device scalars read inside the step (a captured step follows their
    // writes): Adam's learning rate and the loss's entropy coefficient
    // (the reference's lr_ptr and ppo_bufs.ent_coef, pufferlib.cu:1912-1948)
    double* lr_dev;
    float* ent_dev;
    // rollout policies: models on the same weights with inference
    // activations (reg_rollout), one per env buffer so that buffers' forwards
    // may overlap on their own streams (the reference's per-buffer threads,
    // pufferlib.cu:502-509); made on first use, rolls[b] for roll_n[b] rows
    std::vector<PtcgModel*> rolls;
    std::vector<int> roll_n;
    int prec = 0;
    int sync_free = 0;
    int skip_masked = 1;   // the PPO loss and the sampler mask those slots
    int sampler = 0;       // rollout draws: 0 = inverse CDF (the reference's), 1 = Gumbel-max
    const float* prio = nullptr;   // policy-loss importance weights per rollout row
    PtcgMuon* muon = nullptr;      // optimizer 1 (Muon); nullptr = Adam
    // captured training step (sync-free mode): graph over fixed buffers
    hipStream_t cap_stream = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    // captured rollout steps, one per slot (the reference's per-(t, buf)
    // graphs), and the rollout policy each was captured on
    std::vector<hipGraphExec_t> roll_exec;
    std::vector<int> roll_exec_buf;
    double wd_1d = 0.0;
    int64_t global_step = 0, epoch = 0;
    // phase timing (the reference's profile.events, pufferlib.cu:1851-2185):
    // pev[k] is mark k (ptcg_trainer_perf_mark, ptcg_trainer_step),
    // pev_rec[k] whether it was recorded since the last commit; perf_s holds
    // seconds per phase since the last log reset
    hipEvent_t pev[PT_NMARK] = {};
    bool pev_rec[PT_NMARK] = {};
    double perf_s[PTCG_PERF_N] = {};
    std::vector<float> st_f[5];
    std::vector<int32_t> st_i[2];
};

extern "C" void ptcg_trainer_free(PtcgTrainer* t) {
    if (!t) return;
    if (t->model) ptcg_model_free(t->model);
    for (auto r : t->rolls)
        if (r) ptcg_model_free(r);
    if (t->muon) ptcg_muon_free(t->muon);
    for (auto x : t->roll_exec)
        if (x) (void)hipGraphExecDestroy(x);
    if (t->graph_exec) (void)hipGraphExecDestroy(t->graph_exec);
    if (t->graph) (void)hipGraphDestroy(t->graph);
    if (t->cap_stream) (void)hipStreamDestroy(t->cap_stream);
    for (auto e : t->pev)
        if (e) (void)hipEventDestroy(e);
    if (t->mem) (void)hipFree(t->mem);
    delete t;
}

// lr and ent_coef into their device scalars (the reference's per-train
// cudaMemcpy to lr_ptr / ppo_bufs.ent_coef, pufferlib.cu:1933,1947)
static int write_schedule(PtcgTrainer* t, double lr, float ent_coef) {
    double v[2];
    memcpy(&v[0], &lr, sizeof lr);
    float e[2] = {ent_coef, 0.f};
    memcpy(&v[1], e, sizeof e);
    PT_HIP(hipMemcpy(t->lr_dev, v, sizeof v, hipMemcpyHostToDevice));
    return PTCG_OK;
}

// A captured step holds every by-value argument of its launches and every
// buffer address.  Whatever changes one of them drops the graph, so that
// replay_step fails ("no captured step") instead of replaying stale values.
static int drop_step_graph(PtcgTrainer* t) {
    if (t->graph_exec) {
        PT_HIP(hipDeviceSynchronize());
        PT_HIP(hipGraphExecDestroy(t->graph_exec));
        t->graph_exec = nullptr;
    }
    if (t->graph) {
        PT_HIP(hipGraphDestroy(t->graph));
        t->graph = nullptr;
    }
    return PTCG_OK;
}
// buf < 0: every slot; else the slots captured on rollout policy buf
static int drop_rollout_graphs(PtcgTrainer* t, int buf = -1) {
    for (size_t i = 0; i < t->roll_exec.size(); ++i)
        if (t->roll_exec[i] && (buf < 0 || t->roll_exec_buf[i] == buf)) {
            PT_HIP(hipDeviceSynchronize());
            PT_HIP(hipGraphExecDestroy(t->roll_exec[i]));
            t->roll_exec[i] = nullptr;
        }
    return PTCG_OK;
}

extern "C" int ptcg_trainer_create(const PtcgDims* dims, const PtcgHypers* hyp, int minibatch,
                                   PtcgTrainer** out) {
    PT_REQUIRE(dims && hyp && out, "trainer_create: null argument");
    PT_REQUIRE(minibatch >= 2, "trainer_create: minibatch %d < 2", minibatch);
    PtcgTrainer* t = new PtcgTrainer();
    t->dm = *dims;
    t->hyp = *hyp;
    t->B = minibatch;
    t->off = pt_obs_offsets(*dims);
    int r = ptcg_model_create(dims, &t->model);
    if (r != PTCG_OK) { delete t; return r; }
    ptcg_model_set_skip_masked_options(t->model, t->skip_masked);
    t->arena = pt_model_arena(t->model);
    t->packed = ptcg_packed_floats(dims);
    const long A1 = dims->n_opt + 1;
    const long B = minibatch;
    size_t off = 0;
    auto take = [&](long floats) { off = (off + 255) & ~(size_t)255; size_t o = off; off += floats * 4; return o; };
    const size_t oP = take(t->arena), oG = take(t->arena), oM = take(t->arena), oV = take(t->arena);
    const size_t oGrad = take(B * A1), oRatio = take(B), oNv = take(B), oStats = take(16),
                 oGuard = take(4), oGate = take(4), oPart = take(pt_ppo_partial_floats(minibatch)),
                 oAdam = take(pt_adam_ws_floats()), oStep = take(4), oHyp = take(4),
                 oDbg = take(B * t->off.size);
    hipError_t e = hipMalloc(&t->mem, off);
    if (e != hipSuccess) {
        ptcg_set_error("trainer_create: hipMalloc(%zu): %s", off, hipGetErrorString(e));
        ptcg_trainer_free(t);
        return PTCG_ERR_HIP;
    }
    e = hipMemset(t->mem, 0, off);
    if (e != hipSuccess) {
        ptcg_set_error("trainer_create: hipMemset: %s", hipGetErrorString(e));
        ptcg_trainer_free(t);
        return PTCG_ERR_HIP;
    }
    auto F = [&](size_t o) { return reinterpret_cast<float*>(t->mem + o); };
    t->P = F(oP); t->Gr = F(oG); t->M = F(oM); t->V = F(oV);
    t->grad = F(oGrad); t->ratio = F(oRatio); t->newvalue = F(oNv); t->stats = F(oStats);
    t->guard = F(oGuard); t->gate = F(oGate); t->ppo_part = F(oPart); t->adam_ws = F(oAdam);
    t->step = reinterpret_cast<int32_t*>(t->mem + oStep);
    t->lr_dev = reinterpret_cast<double*>(t->mem + oHyp);
    t->ent_dev = F(oHyp) + 2;
    t->dbg_obs = F(oDbg);
    for (auto& ev : t->pev) {
        e = hipEventCreate(&ev);
        if (e != hipSuccess) {
            ptcg_set_error("trainer_create: hipEventCreate: %s", hipGetErrorString(e));
            ptcg_trainer_free(t);
            return PTCG_ERR_HIP;
        }
    }
    // the gate starts open, as the reference's (pufferlib.cu:2732-2734)
    const float one = 1.0f;
    e = hipMemcpy(t->gate, &one, sizeof one, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        ptcg_set_error("trainer_create: gate init: %s", hipGetErrorString(e));
        ptcg_trainer_free(t);
        return PTCG_ERR_HIP;
    }
    r = ptcg_model_bind(t->model, t->P, t->Gr);
    if (r == PTCG_OK) r = ptcg_model_reg_train(t->model, minibatch);
    if (r == PTCG_OK) r = write_schedule(t, hyp->lr, hyp->ent_coef);
    if (r != PTCG_OK) { ptcg_trainer_free(t); return r; }
    *out = t;
    return PTCG_OK;
}

extern "C" int ptcg_trainer_set_hypers(PtcgTrainer* t, const PtcgHypers* hyp) {
    PT_REQUIRE(t && hyp, "set_hypers: null argument");
    const PtcgHypers& o = t->hyp;
    // lr and ent_coef live in device scalars; every other field is a launch
    // argument of the captured step (and Muon's momentum of its kernels)
    const bool baked = o.beta1 != hyp->beta1 || o.beta2 != hyp->beta2 || o.eps != hyp->eps ||
                       o.max_grad_norm != hyp->max_grad_norm || o.clip_coef != hyp->clip_coef ||
                       o.vf_clip_coef != hyp->vf_clip_coef || o.vf_coef != hyp->vf_coef ||
                       o.kl_skip_threshold != hyp->kl_skip_threshold ||
                       o.vf_skip_threshold != hyp->vf_skip_threshold;
    if (baked) PT_TRY(drop_step_graph(t));
    PT_TRY(write_schedule(t, hyp->lr, hyp->ent_coef));
    t->hyp = *hyp;
    if (t->muon) {
        PT_TRY(ptcg_muon_set_lr(t->muon, (float)hyp->lr));
        PT_TRY(pt_muon_set_momentum(t->muon, hyp->beta1));
    }
    return PTCG_OK;
}

extern "C" int ptcg_trainer_hyper_ptrs(PtcgTrainer* t, double** lr, float** ent_coef) {
    PT_REQUIRE(t, "hyper_ptrs: null trainer");
    if (lr) *lr = t->lr_dev;
    if (ent_coef) *ent_coef = t->ent_dev;
    return PTCG_OK;
}

extern "C" int ptcg_trainer_set_optimizer(PtcgTrainer* t, int kind, double wd_1d) {
    PT_REQUIRE(t, "set_optimizer: null trainer");
    PT_REQUIRE(kind == 0 || kind == 1, "set_optimizer: kind %d (0 Adam, 1 Muon)", kind);
    PT_TRY(drop_step_graph(t));   // the graph points into the old optimizer's memory
    if (t->muon) {
        ptcg_muon_free(t->muon);
        t->muon = nullptr;
    }
    t->wd_1d = wd_1d;
    if (kind == 1) PT_TRY(ptcg_muon_create(&t->dm, t->hyp.lr, t->hyp.beta1, 0.0, wd_1d, &t->muon));
    return PTCG_OK;
}

extern "C" int ptcg_trainer_set_counters(PtcgTrainer* t, int64_t global_step, int64_t epoch) {
    PT_REQUIRE(t, "set_counters: null trainer");
    t->global_step = global_step;
    t->epoch = epoch;
    return PTCG_OK;
}

extern "C" int ptcg_trainer_get_counters(PtcgTrainer* t, int64_t* global_step, int64_t* epoch) {
    PT_REQUIRE(t, "get_counters: null trainer");
    if (global_step) *global_step = t->global_step;
    if (epoch) *epoch = t->epoch;
    return PTCG_OK;
}

static int arena_copy_in(PtcgTrainer* t, float* dev, const float* packed) {
    std::vector<float> img(t->arena, 0.f);
    PT_TRY(ptcg_packed_to_arena(&t->dm, packed, img.data()));
    PT_HIP(hipMemcpy(dev, img.data(), t->arena * sizeof(float), hipMemcpyHostToDevice));
    return PTCG_OK;
}
static int arena_copy_out(PtcgTrainer* t, const float* dev, float* packed) {
    std::vector<float> img(t->arena);
    PT_HIP(hipDeviceSynchronize());
    PT_HIP(hipMemcpy(img.data(), dev, t->arena * sizeof(float), hipMemcpyDeviceToHost));
    return ptcg_arena_to_packed(&t->dm, img.data(), packed);
}

extern "C" int ptcg_trainer_set_weights(PtcgTrainer* t, const float* packed) {
    PT_REQUIRE(t && packed, "set_weights: null argument");
    return arena_copy_in(t, t->P, packed);
}
extern "C" int ptcg_trainer_get_weights(PtcgTrainer* t, float* packed) {
    PT_REQUIRE(t && packed, "get_weights: null argument");
    return arena_copy_out(t, t->P, packed);
}
extern "C" int ptcg_trainer_get_grads(PtcgTrainer* t, float* packed) {
    PT_REQUIRE(t && packed, "get_grads: null argument");
    return arena_copy_out(t, t->Gr, packed);
}
extern "C" int ptcg_trainer_get_moments(PtcgTrainer* t, float* m, float* v) {
    PT_REQUIRE(t && m && v, "get_moments: null argument");
    PT_TRY(arena_copy_out(t, t->M, m));
    return arena_copy_out(t, t->V, v);
}

// bindings.cu:202-215 (save) / 339-367 (load): packed fp32 blob on disk
extern "C" int ptcg_trainer_save_weights(PtcgTrainer* t, const char* path) {
    PT_REQUIRE(t && path, "save_weights: null argument");
    std::vector<float> packed(t->packed);
    PT_TRY(ptcg_trainer_get_weights(t, packed.data()));
    FILE* f = fopen(path, "wb");
    if (!f) { ptcg_set_error("Failed to open %s for writing", path); return PTCG_ERR_IO; }
    size_t w = fwrite(packed.data(), sizeof(float), packed.size(), f);
    fclose(f);
    if (w != packed.size()) { ptcg_set_error("Failed to write %s", path); return PTCG_ERR_IO; }
    return PTCG_OK;
}

extern "C" int ptcg_trainer_load_weights(PtcgTrainer* t, const char* path) {
    PT_REQUIRE(t && path, "load_weights: null argument");
    FILE* f = fopen(path, "rb");
    if (!f) { ptcg_set_error("Failed to open %s for reading", path); return PTCG_ERR_IO; }
    fseek(f, 0, SEEK_END);
    long size = ftell(f);
    fseek(f, 0, SEEK_SET);
    const long want = t->packed * (long)sizeof(float);
    if (size != want) {
        fclose(f);
        ptcg_set_error("Weight file size mismatch: expected %ld bytes, got %ld", want, size);
        return PTCG_ERR_IO;
    }
    std::vector<float> packed(t->packed);
    size_t rd = fread(packed.data(), 1, want, f);
    fclose(f);
    if ((long)rd != want) { ptcg_set_error("Failed to read weight file %s", path); return PTCG_ERR_IO; }
    return ptcg_trainer_set_weights(t, packed.data());
}

// Adam state: "PTCGADM1" | int64 step | int64 n_params | weights | m | v (packed).
// A separate magic from the reference's Muon state (PTCGSTA1, bindings.cu:257-293).
struct AdmHeader { char magic[8]; int64_t step; int64_t n_params; };
// Muon state, the reference's layout (bindings.cu:257-262): magic, global
// step, epoch, packed count, then packed weights and packed momentum.
struct StaHeader { char magic[8]; int64_t global_step; int64_t epoch; int64_t n_params; };

static int save_state_muon(PtcgTrainer* t, const char* path) {
    std::vector<float> w(t->packed), m(t->packed);
    PT_TRY(arena_copy_out(t, t->P, w.data()));
    PT_TRY(arena_copy_out(t, ptcg_muon_momentum(t->muon), m.data()));
    StaHeader h;
    memcpy(h.magic, "PTCGSTA1", 8);
    h.global_step = t->global_step;
    h.epoch = t->epoch;
    h.n_params = t->packed;
    std::string tmp = std::string(path) + ".tmp";
    FILE* f = fopen(tmp.c_str(), "wb");
    if (!f) { ptcg_set_error("Failed to open %s for writing", tmp.c_str()); return PTCG_ERR_IO; }
    bool ok = fwrite(&h, sizeof h, 1, f) == 1 && fwrite(w.data(), 4, w.size(), f) == w.size() &&
              fwrite(m.data(), 4, m.size(), f) == m.size();
    ok = ok && fflush(f) == 0;
    fclose(f);
    if (!ok || rename(tmp.c_str(), path) != 0) {
        ptcg_set_error("Failed to write state %s", path);
        return PTCG_ERR_IO;
    }
    return PTCG_OK;
}

static int load_state_muon(PtcgTrainer* t, const char* path) {
    FILE* f = fopen(path, "rb");
    if (!f) { ptcg_set_error("Failed to open %s for reading", path); return PTCG_ERR_IO; }
    StaHeader h;
    if (fread(&h, sizeof h, 1, f) != 1 || memcmp(h.magic, "PTCGSTA1", 8) != 0) {
        fclose(f);
        ptcg_set_error("%s is not a PTCGSTA1 state file", path);
        return PTCG_ERR_IO;
    }
    if (h.n_params != t->packed) {
        fclose(f);
        ptcg_set_error("State param count mismatch: file %lld, model %ld", (long long)h.n_params, t->packed);
        return PTCG_ERR_IO;
    }
    std::vector<float> w(t->packed), m(t->packed);
    const bool ok = fread(w.data(), 4, w.size(), f) == w.size() && fread(m.data(), 4, m.size(), f) == m.size();
    fclose(f);
    if (!ok) { ptcg_set_error("Truncated state file %s", path); return PTCG_ERR_IO; }
    PT_TRY(arena_copy_in(t, t->P, w.data()));
    PT_TRY(arena_copy_in(t, ptcg_muon_momentum(t->muon), m.data()));
    PT_HIP(hipDeviceSynchronize());
    t->global_step = h.global_step;
    t->epoch = h.epoch;
    return PTCG_OK;
}

extern "C" int ptcg_trainer_save_state(PtcgTrainer* t, const char* path) {
    PT_REQUIRE(t && path, "save_state: null argument");
    if (t->muon) return save_state_muon(t, path);
    std::vector<float> w(t->packed), m(t->packed), v(t->packed);
    PT_TRY(arena_copy_out(t, t->P, w.data()));
    PT_TRY(arena_copy_out(t, t->M, m.data()));
    PT_TRY(arena_copy_out(t, t->V, v.data()));
    int32_t step = 0;
    PT_HIP(hipMemcpy(&step, t->step, sizeof step, hipMemcpyDeviceToHost));
    AdmHeader h;
    memcpy(h.magic, "PTCGADM1", 8);
    h.step = step;
    h.n_params = t->packed;
    std::string tmp = std::string(path) + ".tmp";
    FILE* f = fopen(tmp.c_str(), "wb");
    if (!f) { ptcg_set_error("Failed to open %s for writing", tmp.c_str()); return PTCG_ERR_IO; }
    bool ok = fwrite(&h, sizeof h, 1, f) == 1 && fwrite(w.data(), 4, w.size(), f) == w.size() &&
              fwrite(m.data(), 4, m.size(), f) == m.size() && fwrite(v.data(), 4, v.size(), f) == v.size();
    ok = ok && fflush(f) == 0;
    fclose(f);
    if (!ok || rename(tmp.c_str(), path) != 0) {
        ptcg_set_error("Failed to write state %s", path);
        return PTCG_ERR_IO;
    }
    return PTCG_OK;
}

extern "C" int ptcg_trainer_load_state(PtcgTrainer* t, const char* path) {
    PT_REQUIRE(t && path, "load_state: null argument");
    if (t->muon) return load_state_muon(t, path);
    FILE* f = fopen(path, "rb");
    if (!f) { ptcg_set_error("Failed to open %s for reading", path); return PTCG_ERR_IO; }
    AdmHeader h;
    if (fread(&h, sizeof h, 1, f) != 1 || memcmp(h.magic, "PTCGADM1", 8) != 0) {
        fclose(f);
        ptcg_set_error("%s is not a PTCGADM1 state file", path);
        return PTCG_ERR_IO;
    }
    if (h.n_params != t->packed) {
        fclose(f);
        ptcg_set_error("State param count mismatch: file %lld, model %ld", (long long)h.n_params, t->packed);
        return PTCG_ERR_IO;
    }
    std::vector<float> w(t->packed), m(t->packed), v(t->packed);
    bool ok = fread(w.data(), 4, w.size(), f) == w.size() && fread(m.data(), 4, m.size(), f) == m.size() &&
              fread(v.data(), 4, v.size(), f) == v.size();
    fclose(f);
    if (!ok) { ptcg_set_error("Truncated state file %s", path); return PTCG_ERR_IO; }
    PT_TRY(arena_copy_in(t, t->P, w.data()));
    PT_TRY(arena_copy_in(t, t->M, m.data()));
    PT_TRY(arena_copy_in(t, t->V, v.data()));
    int32_t step = (int32_t)h.step;
    PT_HIP(hipMemcpy(t->step, &step, sizeof step, hipMemcpyHostToDevice));
    return PTCG_OK;
}

extern "C" int ptcg_trainer_debug_forward(PtcgTrainer* t, const float* obs_host, int n, float* out_host) {
    PT_REQUIRE(t && obs_host && out_host, "debug_forward: null argument");
    PT_REQUIRE(n == t->B, "debug_forward: need exactly %ld floats (minibatch %d x obs %d), got %ld",
               (long)t->B * t->off.size, t->B, t->off.size, (long)n * t->off.size);
    PT_HIP(hipMemcpy(t->dbg_obs, obs_host, (size_t)n * t->off.size * sizeof(float), hipMemcpyHostToDevice));
    float* out = nullptr;
    // debug_forward reports every slot's score, as the reference's does
    PT_TRY(ptcg_model_set_skip_masked_options(t->model, 0));
    const int rf = ptcg_model_forward(t->model, t->dbg_obs, nullptr, n, &out, nullptr);
    PT_TRY(ptcg_model_set_skip_masked_options(t->model, t->skip_masked));
    PT_TRY(rf);
    PT_HIP(hipStreamSynchronize(nullptr));
    PT_HIP(hipMemcpy(out_host, out, (size_t)n * (t->dm.n_opt + 1) * sizeof(float), hipMemcpyDeviceToHost));
    return PTCG_OK;
}

// record phase mark k on stream s (timed: an eager step on a stream that is
// not being captured)
static int perf_rec(PtcgTrainer* t, int k, hipStream_t s, bool timed) {
    if (!timed) return PTCG_OK;
    PT_HIP(hipEventRecord(t->pev[k], s));
    t->pev_rec[k] = true;
    return PTCG_OK;
}

// forward -> PPO loss -> backward (-> gate -> optimizer), the reference's
// minibatch order (pufferlib.cu:2039-2105)
static int step_impl(PtcgTrainer* t, const float* obs, const int32_t* row_idx, const float* actions,
                     const float* old_logprobs, const float* advantages, const float* returns, const float* values,
                     hipStream_t s, bool timed, bool optimizer = true) {
    PT_REQUIRE(t && obs && actions && old_logprobs && advantages && returns && values,
               "trainer_step: null input");
    PT_TRY(perf_rec(t, 3, s, timed));
    float* out = nullptr;
    PT_TRY(ptcg_model_forward(t->model, obs, row_idx, t->B, &out, s));
    PT_TRY(perf_rec(t, 4, s, timed));
    const PtcgHypers& h = t->hyp;
    PT_TRY(pt_ppo_loss(out, t->B, t->dm.n_opt, obs + t->off.opt_mask, t->off.size, row_idx, actions,
                       old_logprobs, advantages, returns, values, t->prio, h.clip_coef, h.vf_clip_coef,
                       h.vf_coef, t->ent_dev, t->grad, t->ratio, t->newvalue, t->stats, t->guard,
                       t->ppo_part, s));
    PT_TRY(perf_rec(t, 5, s, timed));
    PT_TRY(ptcg_model_bind_returns(t->model, returns));
    PT_TRY(ptcg_model_backward(t->model, t->grad, s));
    PT_TRY(perf_rec(t, 6, s, timed));
    if (!optimizer) return PTCG_OK;
    const bool gate_on = h.kl_skip_threshold > 0.f || h.vf_skip_threshold > 0.f;
    if (gate_on)
        PT_TRY(pt_kl_gate(t->guard, h.kl_skip_threshold, h.vf_skip_threshold, t->gate, t->stats + PT_ST_SKIP, s));
    if (t->muon)
        PT_TRY(ptcg_muon_step(t->muon, t->P, t->Gr, h.max_grad_norm, gate_on ? t->gate : nullptr,
                              t->stats + PT_ST_NORM, s));
    else
        PT_TRY(pt_adam_step(t->P, t->Gr, t->M, t->V, t->arena, t->lr_dev, h.beta1, h.beta2, h.eps, h.max_grad_norm,
                            gate_on ? t->gate : nullptr, t->step, t->stats + PT_ST_NORM, t->adam_ws, s));
    PT_TRY(perf_rec(t, 7, s, timed));
    return PTCG_OK;
}

extern "C" int ptcg_trainer_set_prio(PtcgTrainer* t, const float* prio) {
    PT_REQUIRE(t, "trainer_set_prio: null trainer");
    if (prio != t->prio) PT_TRY(drop_step_graph(t));
    t->prio = prio;
    return PTCG_OK;
}

extern "C" int ptcg_trainer_forward_backward(PtcgTrainer* t, const float* obs, const int32_t* row_idx,
                                             const float* actions, const float* old_logprobs,
                                             const float* advantages, const float* returns,
                                             const float* values, void* stream) {
    PT_REQUIRE(t, "trainer_forward_backward: null trainer");
    return step_impl(t, obs, row_idx, actions, old_logprobs, advantages, returns, values, (hipStream_t)stream,
                     false, false);
}

extern "C" int ptcg_trainer_set_static(PtcgTrainer* t, const float* card_static, const float* att_static,
                                       const float* card_text, const float* att_text, const float* skill_text,
                                       const int32_t* card_attacks, const int32_t* card_skills) {
    PT_REQUIRE(t, "trainer_set_static: null trainer");
    PT_TRY(ptcg_model_set_static(t->model, card_static, att_static, card_text, att_text, skill_text,
                                 card_attacks, card_skills));
    // host copies for the rollout policy's own upload
    const PtcgDims& d = t->dm;
    const long NC = d.n_cards, NA = d.n_attacks, NS = d.n_skills;
    t->st_f[0].assign(card_static, card_static + NC * PT_CARD_STATIC);
    t->st_f[1].assign(att_static, att_static + NA * PT_ATT_STATIC);
    t->st_f[2].assign(card_text, card_text + NC * PT_CARD_TEXT);
    t->st_f[3].assign(att_text, att_text + NA * PT_ATT_TEXT);
    t->st_f[4].assign(skill_text, skill_text + NS * PT_SKILL_TEXT);
    t->st_i[0].assign(card_attacks, card_attacks + NC * PT_K_ATT);
    t->st_i[1].assign(card_skills, card_skills + NC * PT_K_SK);
    for (auto r : t->rolls)
        if (r) PT_TRY(ptcg_model_set_static(r, card_static, att_static, card_text, att_text, skill_text,
                                            card_attacks, card_skills));
    return PTCG_OK;
}

extern "C" int ptcg_trainer_set_precision(PtcgTrainer* t, int prec) {
    PT_REQUIRE(t, "trainer_set_precision: null trainer");
    PT_TRY(drop_step_graph(t));
    PT_TRY(drop_rollout_graphs(t));
    PT_TRY(ptcg_model_set_precision(t->model, prec));
    for (auto r : t->rolls)
        if (r) PT_TRY(ptcg_model_set_precision(r, prec));
    t->prec = prec;
    return PTCG_OK;
}

extern "C" int ptcg_trainer_set_skip_masked_options(PtcgTrainer* t, int on) {
    PT_REQUIRE(t, "trainer_set_skip_masked_options: null trainer");
    PT_TRY(drop_step_graph(t));
    PT_TRY(drop_rollout_graphs(t));
    PT_TRY(ptcg_model_set_skip_masked_options(t->model, on));
    for (auto r : t->rolls)
        if (r) PT_TRY(ptcg_model_set_skip_masked_options(r, on));
    t->skip_masked = on != 0;
    return PTCG_OK;
}

extern "C" int ptcg_trainer_set_sync_free(PtcgTrainer* t, int on) {
    PT_REQUIRE(t, "trainer_set_sync_free: null trainer");
    PT_TRY(drop_step_graph(t));
    PT_TRY(drop_rollout_graphs(t));
    PT_TRY(ptcg_model_set_sync_free(t->model, on));
    for (auto r : t->rolls)
        if (r) PT_TRY(ptcg_model_set_sync_free(r, on));
    t->sync_free = on;
    return PTCG_OK;
}

constexpr int PT_MAX_ROLL_BUFS = 64;

// rollout policy `buf`, registered for n rows (allocations happen here,
// never inside a capture)
static int roll_model(PtcgTrainer* t, int buf, int n) {
    PT_REQUIRE(buf >= 0 && buf < PT_MAX_ROLL_BUFS, "rollout: buffer %d outside [0, %d)", buf, PT_MAX_ROLL_BUFS);
    if ((int)t->rolls.size() <= buf) {
        t->rolls.resize(buf + 1, nullptr);
        t->roll_n.resize(buf + 1, 0);
    }
    PtcgModel*& m = t->rolls[buf];
    if (!m || t->roll_n[buf] != n) {
        if (!m) {
            PT_TRY(ptcg_model_create(&t->dm, &m));
            PT_TRY(ptcg_model_bind(m, t->P, t->Gr));
            PT_TRY(ptcg_model_set_precision(m, t->prec));
            PT_TRY(ptcg_model_set_sync_free(m, t->sync_free));
            PT_TRY(ptcg_model_set_skip_masked_options(m, t->skip_masked));
            if (t->dm.tables == 1 && !t->st_i[0].empty())
                PT_TRY(ptcg_model_set_static(m, t->st_f[0].data(), t->st_f[1].data(), t->st_f[2].data(),
                                             t->st_f[3].data(), t->st_f[4].data(), t->st_i[0].data(),
                                             t->st_i[1].data()));
        }
        // captured rollout graphs of this policy hold its old activation buffers: drop them
        PT_TRY(drop_rollout_graphs(t, buf));
        PT_TRY(ptcg_model_reg_rollout(m, n));
        t->roll_n[buf] = n;
    }
    return PTCG_OK;
}

extern "C" int ptcg_trainer_obs_size(PtcgTrainer* t) { return t ? t->off.size : 0; }

static int draw(PtcgTrainer* t, const float* out, const float* obs, const int32_t* row_idx, int n, uint64_t seed,
                uint64_t step, uint64_t* step_dev, float* actions, float* logprobs, float* values, hipStream_t s) {
    const float* mask = obs + t->off.opt_mask;
    if (t->sampler == 1)
        return pt_sample_gumbel(out, n, t->dm.n_opt, mask, t->off.size, row_idx, nullptr, seed, step, step_dev,
                                actions, logprobs, values, nullptr, s);
    if (step_dev)
        return pt_sample_actions_dev(out, n, t->dm.n_opt, mask, t->off.size, row_idx, seed, step_dev, actions,
                                     logprobs, values, s);
    return ptcg_sample_actions(out, n, t->dm.n_opt, mask, t->off.size, row_idx, seed, step, actions, logprobs,
                               values, nullptr, s);
}

extern "C" int ptcg_trainer_rollout_on(PtcgTrainer* t, int buf, const float* obs, const int32_t* row_idx, int n,
                                       uint64_t seed, uint64_t step, float* actions, float* logprobs, float* values,
                                       void* stream) {
    PT_REQUIRE(t && obs && actions && logprobs, "trainer_rollout: null argument");
    PT_REQUIRE(n >= 1, "trainer_rollout: n=%d", n);
    PT_TRY(roll_model(t, buf, n));
    float* out = nullptr;
    PT_TRY(ptcg_model_forward(t->rolls[buf], obs, row_idx, n, &out, stream));
    return draw(t, out, obs, row_idx, n, seed, step, nullptr, actions, logprobs, values, (hipStream_t)stream);
}

extern "C" int ptcg_trainer_rollout(PtcgTrainer* t, const float* obs, const int32_t* row_idx, int n,
                                    uint64_t seed, uint64_t step, float* actions, float* logprobs,
                                    float* values, void* stream) {
    return ptcg_trainer_rollout_on(t, 0, obs, row_idx, n, seed, step, actions, logprobs, values, stream);
}

extern "C" int ptcg_trainer_rollout_output(PtcgTrainer* t, float** dec_out) {
    PT_REQUIRE(t && dec_out, "rollout_output: null argument");
    PT_REQUIRE(!t->rolls.empty() && t->rolls[0], "rollout_output: no rollout has run");
    *dec_out = pt_model_out(t->rolls[0]);
    return PTCG_OK;
}

extern "C" int ptcg_trainer_set_sampler(PtcgTrainer* t, int kind) {
    PT_REQUIRE(t, "set_sampler: null trainer");
    PT_REQUIRE(kind == 0 || kind == 1, "set_sampler: kind %d (0 inverse CDF, 1 Gumbel-max)", kind);
    if (kind != t->sampler) PT_TRY(drop_rollout_graphs(t));
    t->sampler = kind;
    return PTCG_OK;
}

// The reference captures one graph per (time step, buffer) of its rollout
// (net_callback_wrapper, pufferlib.cu:757-946) because each reads and writes
// different rollout slices; the same here: slot k's graph holds the rollout
// forward over its own buffers on rollout policy buf's activations and the
// draw, with the step read from the device counter step_dev and advanced by
// one per replay.  Slots on different policies may replay concurrently on
// different streams.  Sync-free mode.
extern "C" int ptcg_trainer_capture_rollout_on(PtcgTrainer* t, int buf, int slot, const float* obs,
                                               const int32_t* row_idx, int n, uint64_t seed, uint64_t* step_dev,
                                               float* actions, float* logprobs, float* values) {
    PT_REQUIRE(t && obs && actions && logprobs && step_dev, "capture_rollout: null argument");
    PT_REQUIRE(slot >= 0 && slot < 4096, "capture_rollout: slot %d out of range", slot);
    PT_REQUIRE(n >= 1, "capture_rollout: n=%d", n);
    PT_REQUIRE(t->sync_free, "capture_rollout: needs sync-free mode (ptcg_trainer_set_sync_free)");
    PT_TRY(roll_model(t, buf, n));   // allocations happen outside the capture
    if ((int)t->roll_exec.size() <= slot) {
        t->roll_exec.resize(slot + 1, nullptr);
        t->roll_exec_buf.resize(slot + 1, -1);
    }
    if (t->roll_exec[slot]) {
        PT_HIP(hipDeviceSynchronize());
        PT_HIP(hipGraphExecDestroy(t->roll_exec[slot]));
        t->roll_exec[slot] = nullptr;
    }
    if (!t->cap_stream) PT_HIP(hipStreamCreateWithFlags(&t->cap_stream, hipStreamNonBlocking));
    PT_HIP(hipDeviceSynchronize());
    PT_HIP(hipStreamBeginCapture(t->cap_stream, hipStreamCaptureModeThreadLocal));
    float* out = nullptr;
    int r = ptcg_model_forward(t->rolls[buf], obs, row_idx, n, &out, t->cap_stream);
    if (r == PTCG_OK)
        r = draw(t, out, obs, row_idx, n, seed, 0, step_dev, actions, logprobs, values, t->cap_stream);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(t->cap_stream, &g);
    if (r != PTCG_OK) {
        if (g) (void)hipGraphDestroy(g);
        return r;
    }
    PT_HIP(e);
    hipGraphExec_t x = nullptr;
    const hipError_t ei = hipGraphInstantiateWithFlags(&x, g, 0);
    (void)hipGraphDestroy(g);
    PT_HIP(ei);
    t->roll_exec[slot] = x;
    t->roll_exec_buf[slot] = buf;
    return PTCG_OK;
}

extern "C" int ptcg_trainer_capture_rollout(PtcgTrainer* t, int slot, const float* obs, const int32_t* row_idx,
                                            int n, uint64_t seed, uint64_t* step_dev, float* actions,
                                            float* logprobs, float* values) {
    return ptcg_trainer_capture_rollout_on(t, 0, slot, obs, row_idx, n, seed, step_dev, actions, logprobs, values);
}

extern "C" int ptcg_trainer_replay_rollout(PtcgTrainer* t, int slot, void* stream) {
    PT_REQUIRE(t && slot >= 0 && slot < (int)t->roll_exec.size() && t->roll_exec[slot],
               "replay_rollout: slot %d has no captured rollout", slot);
    PT_HIP(hipGraphLaunch(t->roll_exec[slot], (hipStream_t)stream));
    return PTCG_OK;
}

extern "C" int ptcg_trainer_step(PtcgTrainer* t, const float* obs, const int32_t* row_idx,
                                 const float* actions, const float* old_logprobs, const float* advantages,
                                 const float* returns, const float* values, void* stream) {
    PT_REQUIRE(t, "trainer_step: null trainer");
    hipStream_t s = (hipStream_t)stream;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    PT_HIP(hipStreamIsCapturing(s, &cs));
    return step_impl(t, obs, row_idx, actions, old_logprobs, advantages, returns, values, s,
                     cs == hipStreamCaptureStatusNone);
}

extern "C" int ptcg_trainer_perf_mark(PtcgTrainer* t, int mark, void* stream) {
    PT_REQUIRE(t, "perf_mark: null trainer");
    PT_REQUIRE(mark >= 0 && mark <= 2, "perf_mark: mark %d outside [0, 2] (3..7 are the step's own)", mark);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    PT_HIP(hipStreamIsCapturing((hipStream_t)stream, &cs));
    return perf_rec(t, mark, (hipStream_t)stream, cs == hipStreamCaptureStatusNone);
}

// elapsed seconds between marks a and b, 0 unless both were recorded
static int perf_span(PtcgTrainer* t, int a, int b, double* sec) {
    *sec = 0.0;
    if (!t->pev_rec[a] || !t->pev_rec[b]) return PTCG_OK;
    float ms = 0.f;
    PT_HIP(hipEventElapsedTime(&ms, t->pev[a], t->pev[b]));
    *sec = ms > 0.f ? ms * 1e-3 : 0.0;
    return PTCG_OK;
}

extern "C" int ptcg_trainer_perf_commit(PtcgTrainer* t, int minibatches) {
    PT_REQUIRE(t, "perf_commit: null trainer");
    PT_REQUIRE(minibatches >= 0, "perf_commit: minibatches %d < 0", minibatches);
    for (int k = 0; k < PT_NMARK; ++k)
        if (t->pev_rec[k]) PT_HIP(hipEventSynchronize(t->pev[k]));
    double pre, misc, fwd, loss, bwd, opt;
    PT_TRY(perf_span(t, 0, 1, &pre));
    PT_TRY(perf_span(t, 2, 3, &misc));
    PT_TRY(perf_span(t, 3, 4, &fwd));
    PT_TRY(perf_span(t, 4, 5, &loss));
    PT_TRY(perf_span(t, 5, 6, &bwd));
    PT_TRY(perf_span(t, 6, 7, &opt));
    const double mb = (double)minibatches;
    t->perf_s[PTCG_PERF_TRAIN_MISC] += pre + misc * mb;
    t->perf_s[PTCG_PERF_TRAIN_FORWARD] += (fwd + loss + bwd + opt) * mb;
    t->perf_s[PTCG_PERF_FORWARD] += fwd * mb;
    t->perf_s[PTCG_PERF_LOSS] += loss * mb;
    t->perf_s[PTCG_PERF_BACKWARD] += bwd * mb;
    t->perf_s[PTCG_PERF_OPTIMIZER] += opt * mb;
    for (bool& r : t->pev_rec) r = false;
    return PTCG_OK;
}

extern "C" int ptcg_trainer_perf_add(PtcgTrainer* t, int phase, double seconds) {
    PT_REQUIRE(t, "perf_add: null trainer");
    PT_REQUIRE(phase >= 0 && phase < PTCG_PERF_N, "perf_add: phase %d outside [0, %d)", phase, PTCG_PERF_N);
    t->perf_s[phase] += seconds;
    return PTCG_OK;
}

// The reference captures its training step in a CUDA graph after warmup and
// replays it per minibatch over fixed buffers (pufferlib.cu:2019-2140); the
// same here with a HIP graph over the sync-free step (no host read-back, so
// every node is a kernel).  Pointers are baked in: the caller rewrites the
// contents of row_idx (and the per-row arrays) between replays.
extern "C" int ptcg_trainer_capture_step(PtcgTrainer* t, const float* obs, const int32_t* row_idx,
                                         const float* actions, const float* old_logprobs,
                                         const float* advantages, const float* returns, const float* values) {
    PT_REQUIRE(t, "capture_step: null trainer");
    PT_REQUIRE(t->sync_free, "capture_step: needs sync-free mode (ptcg_trainer_set_sync_free)");
    PT_TRY(drop_step_graph(t));
    if (!t->cap_stream) PT_HIP(hipStreamCreateWithFlags(&t->cap_stream, hipStreamNonBlocking));
    PT_HIP(hipDeviceSynchronize());
    PT_HIP(hipStreamBeginCapture(t->cap_stream, hipStreamCaptureModeThreadLocal));
    const int r = step_impl(t, obs, row_idx, actions, old_logprobs, advantages, returns, values, t->cap_stream,
                            false);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(t->cap_stream, &g);
    if (r != PTCG_OK) {
        if (g) (void)hipGraphDestroy(g);
        return r;
    }
    PT_HIP(e);
    t->graph = g;
    PT_HIP(hipGraphInstantiateWithFlags(&t->graph_exec, t->graph, 0));
    return PTCG_OK;
}

extern "C" int ptcg_trainer_replay_step(PtcgTrainer* t, void* stream) {
    PT_REQUIRE(t && t->graph_exec, "replay_step: no captured step (ptcg_trainer_capture_step; a change of "
               "optimizer, mode, gate or a by-value hyper-parameter drops the captured graph)");
    PT_HIP(hipGraphLaunch(t->graph_exec, (hipStream_t)stream));
    return PTCG_OK;
}

// amdgpu's busy percentage of the current device from sysfs (the
// reference reads NVML's utilisation, bindings.cu:92-94); -1 if unreadable
static float gpu_busy_percent() {
    int dev = 0;
    char bus[64] = {0};
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetPCIBusId(bus, sizeof bus, dev) != hipSuccess) return -1.f;
    for (char* c = bus; *c; ++c) *c = (char)tolower((unsigned char)*c);
    char path[160];
    snprintf(path, sizeof path, "/sys/bus/pci/devices/%s/gpu_busy_percent", bus);
    FILE* f = fopen(path, "r");
    if (!f) return -1.f;
    int v = -1;
    if (fscanf(f, "%d", &v) != 1) v = -1;
    fclose(f);
    return (float)v;
}

extern "C" int ptcg_trainer_log(PtcgTrainer* t, PtcgLog* out, int reset) {
    PT_REQUIRE(t && out, "trainer_log: null argument");
    PT_HIP(hipDeviceSynchronize());
    float st[PT_ST_FLOATS];
    PT_HIP(hipMemcpy(st, t->stats, sizeof st, hipMemcpyDeviceToHost));
    double lr = 0.0;
    float ent = 0.f, gate = 1.f;
    // the applied learning rate: the scalar the optimizer's kernels read
    if (t->muon) {
        float lf = 0.f;
        PT_TRY(pt_muon_lr(t->muon, &lf));
        lr = lf;
    } else {
        PT_HIP(hipMemcpy(&lr, t->lr_dev, sizeof lr, hipMemcpyDeviceToHost));
    }
    PT_HIP(hipMemcpy(&ent, t->ent_dev, sizeof ent, hipMemcpyDeviceToHost));
    PT_HIP(hipMemcpy(&gate, t->gate, sizeof gate, hipMemcpyDeviceToHost));
    PtcgLog& o = *out;
    memset(&o, 0, sizeof o);
    for (int i = 0; i < 7; ++i) o.loss[i] = st[i];
    o.n = st[7];
    o.kl_skipped = st[PT_ST_SKIP];
    o.vf_skipped = st[PT_ST_SKIP + 1];
    o.grad_norm = st[PT_ST_NORM];
    o.gate = gate;
    o.lr = (float)lr;
    o.ent_coef = ent;
    o.gpu_percent = gpu_busy_percent();
    for (int i = 0; i < PTCG_PERF_N; ++i) o.perf_s[i] = t->perf_s[i];
    size_t fr = 0, tot = 0;
    PT_HIP(hipMemGetInfo(&fr, &tot));
    const double gib = 1024.0 * 1024.0 * 1024.0;
    o.vram_used_gb = (double)(tot - fr) / gib;
    o.vram_total_gb = (double)tot / gib;
    o.global_step = t->global_step;
    o.epoch = t->epoch;
    if (reset) {
        // the loss sums and both skip counters; the grad norm is overwritten
        // by every step and the gate keeps its last decision
        PT_HIP(hipMemset(t->stats, 0, (PT_ST_SKIP + 2) * sizeof(float)));
        for (double& p : t->perf_s) p = 0.0;
    }
    return PTCG_OK;
}

extern "C" int ptcg_trainer_buffers(PtcgTrainer* t, float** dec_out, float** ppo_grad, float** ratio,
                                    float** newvalue) {
    PT_REQUIRE(t, "buffers: null trainer");
    if (dec_out) *dec_out = pt_model_out(t->model);
    if (ppo_grad) *ppo_grad = t->grad;
    if (ratio) *ratio = t->ratio;
    if (newvalue) *newvalue = t->newvalue;
    return PTCG_OK;
}

extern "C" int ptcg_trainer_sync(PtcgTrainer* t) {
    (void)t;
    PT_HIP(hipDeviceSynchronize());
    return PTCG_OK;
}

extern "C" int ptcg_trainer_step_count(PtcgTrainer* t, int32_t* out) {
    PT_REQUIRE(t && out, "step_count: null argument");
    PT_HIP(hipMemcpy(out, t->step, sizeof(int32_t), hipMemcpyDeviceToHost));
    return PTCG_OK;
}
