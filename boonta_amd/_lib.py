"""ctypes binding of libppo_hip.so (the C ABI declared in include/ppo_hip.h).

The library is the only compute path: if it is missing or a call fails, an
error is raised; nothing falls back to a CPU or PyTorch implementation.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libppo_hip.so")
CSRC = os.path.join(_HERE, "csrc")

P = ctypes.c_void_p
I = ctypes.c_int
I64 = ctypes.c_int64
F = ctypes.c_float
D = ctypes.c_double
SZ = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/ppo_hip.h
SIGNATURES = {
    "ppo_last_error": (ctypes.c_char_p, []),
    "ppo_clear_error": (None, []),
    "ppo_abi_version": (I, []),
    "ppo_device_check": (I, [I]),
    "ppo_event_create": (I, [ctypes.POINTER(ctypes.c_void_p)]),
    "ppo_event_destroy": (I, [P]),
    "ppo_stream_wait": (I, [P, P, P]),
    "ppo_gae_f32": (I, [P, P, P, P, P, P, P, P, P, P, I, I, D, D, I]),
    "ppo_vtrace_f32": (I, [P, P, P, P, P, P, P, I64, F, F, P, P, I, I, D, D, I]),
    "ppo_normalize_workspace": (SZ, [I64]),
    "ppo_normalize_advantages_f32": (I, [P, P, I64, P, SZ]),
    "ppo_pupo_advantages_f32": (I, [P, P, P, I, P, I, I, P]),
    "ppo_fill_f32": (I, [P, P, I64, F]),
    "ppo_threefry_split": (I, [P, P, P, I64]),
    "ppo_permutation_workspace": (SZ, [I64]),
    "ppo_permutation_bucket_bits": (I, [I64]),
    "ppo_permutation_bucket_cap": (I, [I64]),
    "ppo_permutation": (I, [P, P, P, I64, P, SZ]),
    "ppo_epoch_permutations_workspace": (SZ, [I, I64]),
    "ppo_epoch_permutations": (I, [P, P, I, I64, P, P, SZ]),
    "ppo_epoch_permutations_noalloc": (I, [P, P, I, I64, P]),
    "ppo_sample_max_outputs": (I, []),
    "ppo_sample_categorical_f32": (I, [P, P, I64, I, I, P, I64, P, F, P, P, P]),
    "ppo_sample_gaussian_f32": (I, [P, P, I64, P, I64, I, I, P, I64, P, F, P, I64, P, P]),
    "ppo_step_mlp_max_layers": (I, []),
    "ppo_step_mlp_max_obs": (I, []),
    "ppo_step_mlp_categorical_f32": (I, [P, P, I64, I, I, I, P, P, P, I, P, I64, P, I, P, F, P, P, P]),
    "ppo_priority_choice_max_envs": (I, []),
    "ppo_priority_choice_f32": (I, [P, P, I64, I, I, F, F, P, I, P, P, P]),
    "ppo_gemm_ln_act_fwd_f32": (I, [P, P, I64, P, P, I64, P, P, P, P, I64, P, I64, P, P, I, I, I, F, I]),
    "ppo_mlp_chain_max_layers": (I, []),
    "ppo_mlp_ln_fwd_f32": (I, [P, I, I, P, I64, P, I, I, P, I64, I64, P, P, P, P, P, I64, P, P, F, I, I64, I64, I64,
                               I64, P, I64]),
    "ppo_mlp_ln_bwd_blocks": (I, [I]),
    "ppo_mlp_ln_bwd_f32": (I, [P, I, I, P, I64, I, P, P, P, P, P, P, I64, P, I64, P, I, I64, I64, I64, I64, I64]),
    "ppo_gemm_ln_act_fwd_f32_towers": (I, [P, I, P, I64, P, P, I64, P, P, P, P, I64, P, I64, P, P, I, I, I, F, I,
                                           I64, I64, I64, I64]),
    "ppo_mlp16_max_layers": (I, []),
    "ppo_mlp16_ln_fwd": (I, [P, I, P, I64, I64, I, I, P, P, P, P, P, P, P, I64, P, P, F, I, P, P, I, P, I64, I]),
    "ppo_pack_bf16_operands": (I, [P, I, P, I64, I, I, P, P, P, I64, I, I, P, P]),
    "ppo_pack_bf16_operand_padded": (I, [P, P, I64, I, I, I, P, P]),
    "ppo_mlp16_ln_bwd_blocks": (I, [I]),
    "ppo_mlp16_ln_bwd": (I, [P, I, P, I64, I, P, P, P, P, P, P, P, I64, P, I, P, I64, P, I, I, I, P, I64]),
    "ppo_linear_scan_fwd": (I, [P, I, P, P, P, P, I, I, I]),
    "ppo_linear_scan_bwd": (I, [P, I, P, P, P, P, P, P, P, I, I, I]),
    "ppo_ssm_scan_fwd": (I, [P, I, P, P, P, P, P, P, I, I, I]),
    "ppo_ssm_scan_bwd": (I, [P, I, P, P, P, P, P, P, P, P, P, I, I, I]),
    "ppo_gemm_f32": (I, [P, I, I, P, I64, P, P, I64, P, I64, I, I, I, I, I64, I, P, I, P, P, I64, P, I]),
    "ppo_gemm_f32_towers": (I, [P, I, I, I, P, I64, P, P, I64, P, I64, I, I, I, I, I64, I, P, I, P, P, I64, P, I,
                                I64, I64, I64, I64, I64, I64, I64]),
    "ppo_gemm_bf16": (I, [P, I, I, P, I64, P, P, I64, P, I64, I, I, I, I, I64, I, P, I, I, P, I64, P, I]),
    "ppo_round_bf16": (I, [P, P, I64]),
    "ppo_gemm_bf16s": (I, [P, I, I, I, I, P, I64, P, P, I64, P, I64, I, I, I, I, I64, I, P, I, I, P, I64, P, I]),
    "ppo_gemm_bf16s_dw_group": (I, [P, I, P, P, P, P, P, P, P, P, P, P, P, P, P]),
    "ppo_gemm_f32_dw_group": (I, [P, I, P, P, P, P, P, P, P, P, P, P, P, P, P]),
    "ppo_gemm_f32_dw_final_slots": (I, [I, P, P]),
    "ppo_gemm_f32_dw_group_final": (I, [P, I, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, I, I,
                                        I]),
    "ppo_cast_bf16": (I, [P, P, P, I64]),
    "ppo_cast_bf16_2d": (I, [P, P, I64, P, I64, I, I]),
    "ppo_pad_rows_f32": (I, [P, P, I64, P, I64, I, I]),
    "ppo_splits_bias_act_bf16": (I, [P, P, I64, I64, I, P, I, P, I64, I, I]),
    "ppo_layernorm_act_fwd_f32": (I, [P, P, I64, P, P, P, I64, P, P, I, I, F, I]),
    "ppo_layernorm_act_fwd_bf16": (I, [P, P, I64, P, P, P, I64, P, P, I, I, F, I]),
    "ppo_layernorm_act_fwd_bf16_out16": (I, [P, P, I64, P, P, P, I64, P, I64, P, P, I, I, F, I]),
    "ppo_layernorm_act_bwd_bf16": (I, [P, P, I64, P, I64, P, P, P, P, P, I64, P, I, I, I]),
    "ppo_layernorm_act_bwd_bf16_out16": (I, [P, P, I64, P, I64, P, P, P, P, P, I64, P, I, I, I]),
    "ppo_layernorm_bwd_blocks": (I, [I]),
    "ppo_layernorm_act_bwd_f32": (I, [P, P, I64, P, I64, P, P, P, P, P, I64, P, I, I, I]),
    "ppo_layernorm_act_bwd_f32_towers": (I, [P, I, P, I64, P, I64, P, P, P, P, P, I64, P, I, I, I, I64, I64, I64,
                                             I64]),
    "ppo_act_fwd_f32": (I, [P, P, I64, P, I64, I, I, I]),
    "ppo_act_bwd_f32": (I, [P, P, I64, P, I64, P, I64, I, I, I]),
    "ppo_loss_blocks": (I, [I]),
    "ppo_loss_stat_count": (I, []),
    "ppo_loss_f32": (I, [P, I, I, P, P, I64, P, I64, I, P, P, P, P, P, P, P, P, P, P, P, F, I, F, F, F]),
    "ppo_loss_finalize": (I, [P, P, I, I, F, F, P]),
    "ppo_loss_finalize_steps": (I, [P, P, I, I, I, F, F, P]),
    "ppo_head_loss_blocks": (I, [I]),
    "ppo_head_loss_max_outputs": (I, []),
    "ppo_head_loss_max_features": (I, []),
    "ppo_head_loss_f32": (I, [P, I, I, P, P, I64, P, I64, P, I, P, I64, P, I64, P, I, I, P, P, P, P, P, P, P,
                              I, P, I64, P, I64, I, P, I64, P, I64, P, P, P, P, P, P, F, I, F, F, F, I64]),
    "ppo_pack_samples": (I, [P, I64, P, P, P, P, P, P]),
    "ppo_mlp_ln_fwd_head_loss_f32": (I, [P, I, I, P, I64, P, I, I, P, I64, I64, P, P, P, P, P, I64, P, P, F, I, I64,
                                         I64, I64, I64, P, I64,
                                         I, I, P, P, I64, P, I64, P, I, P, I64, P, I64, P, I, I, P, P, P, P, P, P,
                                         P, I, P, I64, P, I64, I, P, I64, P, I64, P, P, P, P, P, P, F, I, F, F, F,
                                         I64]),
    "ppo_mlp_ln_fwd_head_loss_bwd_f32": (I, [P, I, I, P, I64, P, I, I, P, I64, I64, P, P, P, P, P, I64, P, P, F, I,
                                             I64, I64, I64, I64, P, I64,
                                             I, I, P, P, I64, P, I64, P, I, P, I64, P, I64, P, I, I, P, P, P, P, P,
                                             P, P, I, P, I64, P, I64, I, P, I64, P, I64, P, P, P, P, P, P, F, I, F,
                                             F, F, I64, P, P, I64]),
    "ppo_head_loss_ratio_f32": (I, [P, I, I, P, P, I64, P, I64, P, I, P, I64, P, I64, P, I, I, P, P, P, P, P, P, P,
                                    I, P, I64, P, I64, I, P, I64, P, I64, P, P, P, P, P, P, F, I, F, F, F, P, I,
                                    I, I64]),
    "ppo_gru_fwd_step_f32": (I, [P, P, I64, P, I64, P, P, P, P, P, I64, P, P, I64, P, I64, P, I64, I, I]),
    "ppo_gru_bwd_step_f32": (I, [P, P, I64, P, I64, P, I64, P, I64, P, P, P, P, I64, P, I64, P, I64, P, I64, P,
                                 I64, I, I]),
    "ppo_gru_seq_max_workgroups": (I, []),
    "ppo_gru_seq_exchange_bytes": (I64, [I, I]),
    "ppo_gru_fwd_seq_f32": (I, [P, P, I64, I64, P, I64, P, P, P, P, I64, P, I64, P, P, I64, I64, P, I64, I64, P,
                                I64, I64, I, I, I, P, P, I]),
    "ppo_gru_bwd_seq_f32": (I, [P, P, I64, P, P, P, I64, P, I64, I64, P, I64, I64, P, I64, I64, P, I64, I64, P,
                                I64, I64, I, I, I, P, P, I]),
    "ppo_gru_fwd_seq_xw_f32": (I, [P, P, I64, P, P, P, P, I64, P, I64, P, P, I64, I64, P, I64, I64, P, I64, I64,
                                   I, I, I, P, P, I, P, I64, I64, I, P, I64, P, I, P, I64]),
    "ppo_gru_seq_dw_parts": (I, [I]),
    "ppo_gru_bwd_seq_dw_f32": (I, [P, P, I64, P, P, P, I64, P, I64, I64, P, I64, I64, P, I64, I64, P, I64, I64, P,
                                   I64, I64, I, I, I, P, P, I, P, I64, I64, I, P, P, P, P, I, P, I64]),
    "ppo_sequence_rows": (I, [P, P, I, I, I, I, P]),
    "ppo_grad_reduce_segment_bytes": (I, []),
    "ppo_grad_reduce_chunk_bytes": (I, []),
    "ppo_grad_reduce_chunk_elems": (I, []),
    "ppo_grad_reduce_few_parts": (I, []),
    "ppo_grad_reduce_wide_parts": (I, []),
    "ppo_grad_reduce_wide_chunk_elems": (I, []),
    "ppo_grad_reduce": (I, [P, P, P, I, I, I, P]),
    "ppo_sumsq_total": (I, [P, P, I, P]),
    "ppo_adam_clip_f32": (I, [P, P, P, P, P, P, I64, P, I, D, D, D, D, D, P, I, P]),
    "ppo_adam_clip_wt_f32": (I, [P, P, P, P, P, P, I64, P, I, D, D, D, D, D, P, I, P, I, P, P]),
    "ppo_count_advance": (I, [P, P, I, P]),
}

ACT = {"none": 0, None: 0, "relu": 1, "tanh": 2, "silu": 3}
DIST = {"categorical": 0, "gaussian": 1}

_lib = None


class KernelError(RuntimeError):
    pass


def build(verbose: bool = False, force: bool = False) -> str:
    """Compiles the HIP sources for gfx950 into boonta_amd/libppo_hip.so
    (force: every source again, also where the built files are current)."""
    jobs = str(min(16, os.cpu_count() or 4))
    out = subprocess.run(["make", "-C", CSRC, "-j", jobs] + (["-B"] if force else []), capture_output=not verbose,
                         text=True)
    if out.returncode != 0:
        raise KernelError(f"building libppo_hip.so failed:\n{out.stdout}\n{out.stderr}")
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Loads the library (it must already be built; see build())."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise KernelError(f"{LIB_PATH} is missing: build it with boonta_amd._lib.build() "
                          "(hipcc --offload-arch=gfx950); there is no fallback path")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def call(name: str, *args) -> int:
    """Calls an int-returning entry point and raises on a negative status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.ppo_last_error().decode(errors="replace")
        raise KernelError(f"{name} failed ({rc}): {msg}")
    return rc


def exported_symbols() -> list[str]:
    return list(SIGNATURES)
