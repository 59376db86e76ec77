"""ctypes binding of libptcg_amd.so (the C ABI in include/ptcg_amd.h).

The library is the only compute path: if it is missing or fails to load,
every entry point raises — there is no CPU fallback.
"""
import ctypes
import os

from .dims import CPtcgDims

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libptcg_amd.so")

c_float_p = ctypes.POINTER(ctypes.c_float)
c_i32_p = ctypes.POINTER(ctypes.c_int32)
c_void_p = ctypes.c_void_p


class CPtcgHypers(ctypes.Structure):
    _fields_ = [(n, ctypes.c_double) for n in ("lr", "beta1", "beta2", "eps")] + \
        [(n, ctypes.c_float) for n in (
            "max_grad_norm", "clip_coef", "vf_clip_coef", "vf_coef", "ent_coef",
            "kl_skip_threshold", "vf_skip_threshold")]


PERF_N = 9   # PTCG_PERF_N


class CPtcgLog(ctypes.Structure):
    """struct PtcgLog of include/ptcg_amd.h (ptcg_trainer_log)."""
    _fields_ = [("loss", ctypes.c_float * 7)] + \
        [(n, ctypes.c_float) for n in ("n", "kl_skipped", "vf_skipped", "gate", "grad_norm", "lr", "ent_coef",
                                       "gpu_percent", "pad_")] + \
        [("perf_s", ctypes.c_double * PERF_N), ("vram_used_gb", ctypes.c_double),
         ("vram_total_gb", ctypes.c_double), ("global_step", ctypes.c_int64), ("epoch", ctypes.c_int64)]


# name -> (restype, argtypes)
_SIGS = {
    "ptcg_last_error": (ctypes.c_char_p, []),
    "ptcg_abi_version": (ctypes.c_int, []),
    "ptcg_obs_size": (ctypes.c_int, [ctypes.POINTER(CPtcgDims)]),
    "ptcg_num_params": (ctypes.c_int, [ctypes.POINTER(CPtcgDims)]),
    "ptcg_param_info": (ctypes.c_int, [ctypes.POINTER(CPtcgDims), ctypes.c_int,
                                       ctypes.POINTER(ctypes.c_char_p),
                                       ctypes.POINTER(ctypes.c_int64),
                                       ctypes.POINTER(ctypes.c_int64)]),
    "ptcg_packed_floats": (ctypes.c_int64, [ctypes.POINTER(CPtcgDims)]),
    "ptcg_arena_floats": (ctypes.c_int64, [ctypes.POINTER(CPtcgDims)]),
    "ptcg_packed_to_arena": (ctypes.c_int, [ctypes.POINTER(CPtcgDims), c_float_p, c_float_p]),
    "ptcg_arena_to_packed": (ctypes.c_int, [ctypes.POINTER(CPtcgDims), c_float_p, c_float_p]),
    "ptcg_model_create": (ctypes.c_int, [ctypes.POINTER(CPtcgDims), ctypes.POINTER(c_void_p)]),
    "ptcg_model_bind": (ctypes.c_int, [c_void_p, c_void_p, c_void_p]),
    "ptcg_model_reg_train": (ctypes.c_int, [c_void_p, ctypes.c_int]),
    "ptcg_model_forward": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, ctypes.c_int,
                                          ctypes.POINTER(c_void_p), c_void_p]),
    "ptcg_model_backward": (ctypes.c_int, [c_void_p, c_void_p, c_void_p]),
    "ptcg_model_dump_stages": (ctypes.c_int, [c_void_p, ctypes.c_char_p, c_void_p]),
    "ptcg_model_set_static": (ctypes.c_int, [c_void_p] * 8),
    "ptcg_model_bind_returns": (ctypes.c_int, [c_void_p, c_void_p]),
    "ptcg_trainer_set_static": (ctypes.c_int, [c_void_p] * 8),
    "ptcg_model_reg_rollout": (ctypes.c_int, [c_void_p, ctypes.c_int]),
    "ptcg_sample_actions": (ctypes.c_int, [c_void_p, ctypes.c_int, ctypes.c_int, c_void_p, ctypes.c_int64,
                                           c_void_p, ctypes.c_uint64, ctypes.c_uint64, c_void_p, c_void_p,
                                           c_void_p, c_void_p, c_void_p]),
    "ptcg_trainer_rollout": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, ctypes.c_int, ctypes.c_uint64,
                                            ctypes.c_uint64, c_void_p, c_void_p, c_void_p, c_void_p]),
    "ptcg_model_set_precision": (ctypes.c_int, [c_void_p, ctypes.c_int]),
    "ptcg_trainer_set_precision": (ctypes.c_int, [c_void_p, ctypes.c_int]),
    "ptcg_model_set_sync_free": (ctypes.c_int, [c_void_p, ctypes.c_int]),
    "ptcg_trainer_set_sync_free": (ctypes.c_int, [c_void_p, ctypes.c_int]),
    "ptcg_model_set_skip_masked_options": (ctypes.c_int, [c_void_p, ctypes.c_int]),
    "ptcg_trainer_set_skip_masked_options": (ctypes.c_int, [c_void_p, ctypes.c_int]),
    "ptcg_model_free": (None, [c_void_p]),
    "ptcg_ppo_loss_fwd_bwd": (ctypes.c_int, [
        c_void_p, ctypes.c_int, ctypes.c_int, c_void_p, ctypes.c_int64, c_void_p,
        c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
        ctypes.c_float, ctypes.c_float, ctypes.c_float, c_void_p,
        c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "ptcg_ppo_loss_fwd_bwd_noalloc": (ctypes.c_int, [
        c_void_p, ctypes.c_int, ctypes.c_int, c_void_p, ctypes.c_int64, c_void_p,
        c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
        ctypes.c_float, ctypes.c_float, ctypes.c_float, c_void_p,
        c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "ptcg_sample_actions_gumbel": (ctypes.c_int, [
        c_void_p, ctypes.c_int, ctypes.c_int, c_void_p, ctypes.c_int64, c_void_p, c_void_p,
        ctypes.c_uint64, ctypes.c_uint64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "ptcg_trainer_set_sampler": (ctypes.c_int, [c_void_p, ctypes.c_int]),
    "ptcg_trainer_rollout_output": (ctypes.c_int, [c_void_p, c_void_p]),
    "ptcg_kl_gate": (ctypes.c_int, [c_void_p, ctypes.c_float, ctypes.c_float, c_void_p,
                                    c_void_p, c_void_p]),
    "ptcg_adam_workspace_floats": (ctypes.c_int64, []),
    # lr is a device pointer: a double here, a float in the _lrf variant
    "ptcg_adam_step": (ctypes.c_int, [
        c_void_p, c_void_p, c_void_p, c_void_p, ctypes.c_int64,
        c_void_p, ctypes.c_double, ctypes.c_double, ctypes.c_double, ctypes.c_float,
        c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "ptcg_adam_step_lrf": (ctypes.c_int, [
        c_void_p, c_void_p, c_void_p, c_void_p, ctypes.c_int64,
        c_void_p, ctypes.c_double, ctypes.c_double, ctypes.c_double, ctypes.c_float,
        c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    # device memory
    "ptcg_device_count": (ctypes.c_int, [ctypes.POINTER(ctypes.c_int)]),
    "ptcg_device_alloc": (ctypes.c_int, [ctypes.c_int64, ctypes.POINTER(c_void_p)]),
    "ptcg_device_free": (ctypes.c_int, [c_void_p]),
    "ptcg_memcpy": (ctypes.c_int, [c_void_p, c_void_p, ctypes.c_int64, ctypes.c_int, c_void_p]),
    "ptcg_device_synchronize": (ctypes.c_int, []),
    "ptcg_event_create": (ctypes.c_int, [ctypes.POINTER(c_void_p)]),
    "ptcg_event_record": (ctypes.c_int, [c_void_p, c_void_p]),
    "ptcg_event_elapsed_ms": (ctypes.c_int, [c_void_p, c_void_p, ctypes.POINTER(ctypes.c_float)]),
    "ptcg_event_destroy": (ctypes.c_int, [c_void_p]),
    "ptcg_trainer_create": (ctypes.c_int, [ctypes.POINTER(CPtcgDims), ctypes.POINTER(CPtcgHypers),
                                           ctypes.c_int, ctypes.POINTER(c_void_p)]),
    "ptcg_trainer_free": (None, [c_void_p]),
    "ptcg_trainer_set_hypers": (ctypes.c_int, [c_void_p, ctypes.POINTER(CPtcgHypers)]),
    "ptcg_trainer_hyper_ptrs": (ctypes.c_int, [c_void_p, c_void_p, c_void_p]),
    "ptcg_trainer_set_weights": (ctypes.c_int, [c_void_p, c_float_p]),
    "ptcg_trainer_get_weights": (ctypes.c_int, [c_void_p, c_float_p]),
    "ptcg_trainer_get_grads": (ctypes.c_int, [c_void_p, c_float_p]),
    "ptcg_trainer_get_moments": (ctypes.c_int, [c_void_p, c_float_p, c_float_p]),
    "ptcg_trainer_load_weights": (ctypes.c_int, [c_void_p, ctypes.c_char_p]),
    "ptcg_trainer_save_weights": (ctypes.c_int, [c_void_p, ctypes.c_char_p]),
    "ptcg_trainer_save_state": (ctypes.c_int, [c_void_p, ctypes.c_char_p]),
    "ptcg_trainer_load_state": (ctypes.c_int, [c_void_p, ctypes.c_char_p]),
    "ptcg_trainer_debug_forward": (ctypes.c_int, [c_void_p, c_float_p, ctypes.c_int, c_float_p]),
    "ptcg_trainer_step": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                         c_void_p, c_void_p, c_void_p, c_void_p]),
    "ptcg_trainer_forward_backward": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_void_p,
                                                     c_void_p, c_void_p, c_void_p, c_void_p,
                                                     c_void_p]),
    "ptcg_trainer_log": (ctypes.c_int, [c_void_p, ctypes.POINTER(CPtcgLog), ctypes.c_int]),
    "ptcg_trainer_perf_mark": (ctypes.c_int, [c_void_p, ctypes.c_int, c_void_p]),
    "ptcg_trainer_perf_commit": (ctypes.c_int, [c_void_p, ctypes.c_int]),
    "ptcg_trainer_perf_add": (ctypes.c_int, [c_void_p, ctypes.c_int, ctypes.c_double]),
    "ptcg_trainer_buffers": (ctypes.c_int, [c_void_p, ctypes.POINTER(c_void_p),
                                            ctypes.POINTER(c_void_p), ctypes.POINTER(c_void_p),
                                            ctypes.POINTER(c_void_p)]),
    "ptcg_trainer_sync": (ctypes.c_int, [c_void_p]),
    "ptcg_trainer_step_count": (ctypes.c_int, [c_void_p, c_i32_p]),
    "ptcg_trainer_set_prio": (ctypes.c_int, [c_void_p, c_void_p]),
    "ptcg_trainer_capture_step": (ctypes.c_int, [c_void_p] * 8),
    "ptcg_trainer_replay_step": (ctypes.c_int, [c_void_p, c_void_p]),
    "ptcg_trainer_capture_rollout": (ctypes.c_int, [c_void_p, ctypes.c_int, c_void_p, c_void_p, ctypes.c_int,
                                                    ctypes.c_uint64, c_void_p, c_void_p, c_void_p, c_void_p]),
    "ptcg_trainer_replay_rollout": (ctypes.c_int, [c_void_p, ctypes.c_int, c_void_p]),
    "ptcg_trainer_capture_rollout_on": (ctypes.c_int, [c_void_p, ctypes.c_int, ctypes.c_int, c_void_p, c_void_p,
                                                       ctypes.c_int, ctypes.c_uint64, c_void_p, c_void_p, c_void_p,
                                                       c_void_p]),
    "ptcg_trainer_rollout_on": (ctypes.c_int, [c_void_p, ctypes.c_int, c_void_p, c_void_p, ctypes.c_int,
                                               ctypes.c_uint64, ctypes.c_uint64, c_void_p, c_void_p, c_void_p,
                                               c_void_p]),
    "ptcg_trainer_obs_size": (ctypes.c_int, [c_void_p]),
    "ptcg_transport_create": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                             ctypes.POINTER(c_void_p)]),
    "ptcg_transport_free": (ctypes.c_int, [c_void_p]),
    "ptcg_transport_host": (c_void_p, [c_void_p, ctypes.c_int]),
    "ptcg_transport_device": (c_void_p, [c_void_p, ctypes.c_int]),
    "ptcg_transport_stream": (c_void_p, [c_void_p, ctypes.c_int]),
    "ptcg_transport_agents_per_buffer": (ctypes.c_int, [c_void_p]),
    "ptcg_transport_upload": (ctypes.c_int, [c_void_p, ctypes.c_int]),
    "ptcg_transport_download": (ctypes.c_int, [c_void_p, ctypes.c_int]),
    "ptcg_transport_capture_rollout": (ctypes.c_int, [c_void_p, c_void_p, ctypes.c_int, ctypes.c_int,
                                                      ctypes.c_uint64, c_void_p]),
    "ptcg_transport_step": (ctypes.c_int, [c_void_p, c_void_p, ctypes.c_int, ctypes.c_int]),
    "ptcg_transport_launch": (ctypes.c_int, [c_void_p, c_void_p, ctypes.c_int, ctypes.c_int]),
    "ptcg_transport_wait": (ctypes.c_int, [c_void_p, ctypes.c_int]),
    "ptcg_trainer_set_optimizer": (ctypes.c_int, [c_void_p, ctypes.c_int, ctypes.c_double]),
    "ptcg_trainer_set_counters": (ctypes.c_int, [c_void_p, ctypes.c_int64, ctypes.c_int64]),
    "ptcg_trainer_get_counters": (ctypes.c_int, [c_void_p, ctypes.POINTER(ctypes.c_int64),
                                                 ctypes.POINTER(ctypes.c_int64)]),
    # Muon
    "ptcg_muon_create": (ctypes.c_int, [ctypes.POINTER(CPtcgDims), ctypes.c_double, ctypes.c_double,
                                        ctypes.c_double, ctypes.c_double, ctypes.POINTER(c_void_p)]),
    "ptcg_muon_free": (None, [c_void_p]),
    "ptcg_muon_set_lr": (ctypes.c_int, [c_void_p, ctypes.c_float]),
    "ptcg_muon_momentum": (c_void_p, [c_void_p]),
    "ptcg_muon_step": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, ctypes.c_float, c_void_p, c_void_p,
                                      c_void_p]),
    # rollout-side steps
    "ptcg_transpose_102": (ctypes.c_int, [c_void_p, c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, c_void_p]),
    "ptcg_fill": (ctypes.c_int, [c_void_p, ctypes.c_int64, ctypes.c_float, c_void_p]),
    "ptcg_negamax_advantage": (ctypes.c_int, [
        c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, ctypes.c_int64, ctypes.c_int,
        c_void_p, c_void_p, ctypes.c_float, ctypes.c_float, ctypes.c_float, ctypes.c_float,
        ctypes.c_int, ctypes.c_int, c_void_p]),
    "ptcg_prio_replay_max_segments": (ctypes.c_int, []),
    "ptcg_prio_replay": (ctypes.c_int, [
        c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_float,
        ctypes.c_uint64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "ptcg_index_copy": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                       c_void_p]),
    # include/ptcg_amd_kernels.h
    "ptcg_profile_begin": (ctypes.c_int, [ctypes.c_int]),
    "ptcg_profile_end": (ctypes.c_int, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int),
                                        ctypes.POINTER(ctypes.c_double)]),
    "ptcg_profile_class": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                                          ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_double)]),
    "ptcg_kernel_gemm_axpby": (ctypes.c_int, [
        ctypes.c_int, ctypes.c_int, ctypes.c_int, c_void_p, ctypes.c_int64, ctypes.c_int,
        c_void_p, ctypes.c_int64, ctypes.c_int, c_void_p, ctypes.c_int64, ctypes.c_float,
        c_void_p, ctypes.c_int64, ctypes.c_float, c_void_p]),
    "ptcg_kernel_gemm": (ctypes.c_int, [
        ctypes.c_int, ctypes.c_int, ctypes.c_int, c_void_p, ctypes.c_int64, ctypes.c_int,
        c_void_p, ctypes.c_int64, ctypes.c_int, c_void_p, ctypes.c_int64, ctypes.c_int,
        c_void_p, c_void_p, ctypes.c_int64, c_void_p, ctypes.c_int64, c_void_p,
        ctypes.c_int64, c_void_p]),
    "ptcg_kernel_gemm_rows_dev": (ctypes.c_int, [
        ctypes.c_int, ctypes.c_int, ctypes.c_int, c_void_p, ctypes.c_int64, c_void_p, ctypes.c_int64,
        ctypes.c_int, c_void_p, ctypes.c_int64, ctypes.c_int, c_void_p, c_void_p, ctypes.c_int64, c_void_p,
        ctypes.c_int64, c_void_p, c_void_p, ctypes.c_int64, c_void_p]),
    "ptcg_kernel_gemm_bf16": (ctypes.c_int, [
        ctypes.c_int, ctypes.c_int, ctypes.c_int, c_void_p, ctypes.c_int64, ctypes.c_int,
        c_void_p, ctypes.c_int64, ctypes.c_int, c_void_p, ctypes.c_int64, ctypes.c_int,
        c_void_p, c_void_p, ctypes.c_int64, c_void_p, ctypes.c_int64, c_void_p,
        ctypes.c_int64, c_void_p]),
    "ptcg_kernel_gemm_dw": (ctypes.c_int, [
        ctypes.c_int, ctypes.c_int, ctypes.c_int, c_void_p, ctypes.c_int64, c_void_p, ctypes.c_int64,
        c_void_p, c_void_p, c_void_p, ctypes.c_int64, c_void_p]),
    "ptcg_kernel_gemm_dw_rows_dev": (ctypes.c_int, [
        ctypes.c_int, ctypes.c_int, ctypes.c_int, c_void_p, ctypes.c_int64, c_void_p, ctypes.c_int64,
        c_void_p, c_void_p, c_void_p, c_void_p, ctypes.c_int64, c_void_p]),
    "ptcg_kernel_gemm_dw_bf16": (ctypes.c_int, [
        ctypes.c_int, ctypes.c_int, ctypes.c_int, c_void_p, ctypes.c_int64, c_void_p, ctypes.c_int64,
        c_void_p, c_void_p, c_void_p, ctypes.c_int64, c_void_p]),
    "ptcg_kernel_gemm_bs": (ctypes.c_int, [
        ctypes.c_int, ctypes.c_int, ctypes.c_int, c_void_p, ctypes.c_int64, c_void_p, ctypes.c_int64,
        c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, c_void_p, c_void_p, ctypes.c_int64, c_void_p,
        ctypes.c_int64, c_void_p]),
    "ptcg_kernel_gemm_dw_bs": (ctypes.c_int, [
        ctypes.c_int, ctypes.c_int, ctypes.c_int, c_void_p, ctypes.c_int64, c_void_p, ctypes.c_int64,
        c_void_p, c_void_p, c_void_p, ctypes.c_int64, c_void_p]),
    "ptcg_kernel_attention_path": (ctypes.c_int, [ctypes.c_int, ctypes.c_int]),
    "ptcg_kernel_colsum": (ctypes.c_int, [c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                          c_void_p, c_void_p, ctypes.c_int64, c_void_p]),
    "ptcg_kernel_gemm_resid_ln": (ctypes.c_int, [ctypes.c_int, ctypes.c_int] + [c_void_p] * 10 + [ctypes.c_int]
                                  + [c_void_p] * 2),
    "ptcg_kernel_layernorm_fwd": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_void_p,
                                                 c_void_p, c_void_p, ctypes.c_int, ctypes.c_int,
                                                 c_void_p]),
    "ptcg_kernel_gemm_dx_layernorm_bwd": (ctypes.c_int, [ctypes.c_int, ctypes.c_int] + [c_void_p] * 12
                                          + [ctypes.c_int64] + [c_void_p] * 2),
    "ptcg_kernel_layernorm_bwd": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_void_p,
                                                 c_void_p, c_void_p, c_void_p, c_void_p,
                                                 c_void_p, ctypes.c_int, ctypes.c_int, c_void_p,
                                                 ctypes.c_int64, c_void_p]),
    "ptcg_kernel_attention_fwd": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_void_p,
                                                 ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                 ctypes.c_int, c_void_p]),
    "ptcg_kernel_attention_bwd": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_void_p,
                                                 c_void_p, c_void_p, ctypes.c_int, ctypes.c_int,
                                                 ctypes.c_int, ctypes.c_int, c_void_p]),
    "ptcg_kernel_attention_fwd_bf16": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_void_p,
                                                      ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                      ctypes.c_int, c_void_p]),
    "ptcg_kernel_attention_bwd_bf16": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_void_p,
                                                      c_void_p, c_void_p, ctypes.c_int, ctypes.c_int,
                                                      ctypes.c_int, ctypes.c_int, c_void_p]),
    "ptcg_kernel_attention_bwd_ws_bytes": (ctypes.c_int64, [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                            ctypes.c_int, ctypes.c_int]),
    "ptcg_kernel_attention_bwd_ws": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_void_p,
                                                    c_void_p, c_void_p, ctypes.c_int, ctypes.c_int,
                                                    ctypes.c_int, ctypes.c_int, ctypes.c_int, c_void_p,
                                                    ctypes.c_int64, c_void_p]),
}

_lib = None


def lib():
    """Load the library once; raise if it is absent (no fallback exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} not built: run __graft_entry__.build() (hipcc, gfx950) first")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def exported_symbols():
    return sorted(_SIGS)


class PtcgError(RuntimeError):
    pass


def check(rc):
    if rc != 0:
        raise PtcgError(lib().ptcg_last_error().decode(errors="replace"))
    return rc


def fptr(a):
    """float* of a contiguous float32 numpy array."""
    return a.ctypes.data_as(c_float_p)
