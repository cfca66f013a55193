"""The C ABI library loads without a GPU and exports every entry point that
include/ppo_hip.h declares (no compute call is made here)."""
import ctypes
import os
import re

from boonta_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "ppo_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ppo_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_bound_functions():
    assert set(declared_functions()) == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    missing = [name for name in declared_functions() if not hasattr(lib, name)]
    assert not missing


def test_host_only_entry_points_answer_without_a_device():
    lib = _lib.load()
    assert lib.ppo_abi_version() == 1
    assert lib.ppo_loss_stat_count() == 11
    assert lib.ppo_grad_reduce_segment_bytes() == 40
    assert lib.ppo_grad_reduce_chunk_bytes() == 16
    assert lib.ppo_permutation_workspace(1 << 20) > 3 * 4 * (1 << 20)
    assert lib.ppo_gru_seq_dw_parts(256) == 16 and lib.ppo_gru_seq_dw_parts(17) == 2


def test_argument_errors_are_reported_not_launched():
    lib = _lib.load()
    rc = lib.ppo_gae_f32(None, None, None, None, None, None, None, None, None, None, 4, 4, 0.99, 0.95, 0)
    assert rc == -1
    assert b"null buffer" in lib.ppo_last_error()
    rc = lib.ppo_gemm_f32(None, 0, 0, None, 0, None, None, 0, None, 0, -1, 4, 4, 1, 0, 0, None, 0, None, None,
                          0, None, -1)
    assert rc == -1
    assert lib.ppo_adam_clip_f32(None, None, None, None, None, None, 6, None, 0, 0.5, 1e-3, 0.9, 0.999, 1e-8,
                                 None, 0, None) == -1
    assert lib.ppo_gemm_f32_dw_group(None, 9, None, None, None, None, None, None, None, None, None, None, None, None,
                                     None) == -1   # more problems than a launch takes
    assert lib.ppo_pad_rows_f32(None, None, 87, None, 90, 4, 87) == -1  # a pitch that is not a multiple of 4
    assert b"bad shape" in lib.ppo_last_error()
    assert lib.ppo_gru_bwd_seq_dw_f32(None, None, 768, None, None, None, 0, None, 256, 0, None, 1024, 0, None, 256,
                                      0, None, 256, 0, None, 1024, 0, 16, 256, 4, None, None, 1, None, 256, 0, 256,
                                      None, None, None, None, 0, None, 0) == -1   # no exchange ring


def test_sampling_rejects_unsupported_sizes_without_launching():
    lib = _lib.load()
    big = lib.ppo_sample_max_outputs() + 1
    assert lib.ppo_sample_categorical_f32(None, 1, big, 4, big, None, 0, 1, 1.0, 1, 1, None) == -1
    assert b"ppo_sample_categorical_f32" in lib.ppo_last_error()
    assert lib.ppo_sample_gaussian_f32(None, 1, big, 1, 0, 4, big, None, 0, 1, 1.0, 1, big, 1, None) == -1
    assert lib.ppo_sample_categorical_f32(None, 1, 6, 4, 6, None, 0, None, 1.0, 1, 1, None) == -1


def test_scan_rejects_bad_arguments_without_launching():
    lib = _lib.load()
    assert lib.ppo_linear_scan_fwd(None, 7, 1, 1, 1, 1, 2, 2, 2) == -1
    assert lib.ppo_linear_scan_fwd(None, 0, None, 1, 1, 1, 2, 2, 2) == -1
    assert lib.ppo_linear_scan_bwd(None, 0, 1, 1, 1, 1, None, 1, 1, 2, 2, 2) == -1
    assert lib.ppo_linear_scan_fwd(None, 0, None, None, None, None, 0, 5, 5) == 0


def test_ssm_scan_rejects_missing_done_flags():
    lib = _lib.load()
    assert lib.ppo_ssm_scan_fwd(None, 0, 1, 1, None, None, 1, 1, 2, 2, 2) == -1
    assert lib.ppo_ssm_scan_bwd(None, 0, 1, 1, None, None, 1, 1, 1, 1, 1, 2, 2, 2) == -1


def test_priority_choice_rejects_bad_arguments_without_launching():
    lib = _lib.load()
    big = lib.ppo_priority_choice_max_envs() + 1
    assert lib.ppo_priority_choice_f32(None, 1, big, 4, big, 0.6, 0.4, 1, 4, 1, 1, 1) == -1
    assert b"ppo_priority_choice_f32" in lib.ppo_last_error()
    # the probabilities buffer is required (the weights are read from it)
    assert lib.ppo_priority_choice_f32(None, 1, 8, 4, 8, 0.6, 0.4, 1, 4, 1, 1, None) == -1


def test_one_launch_step_rejects_unsupported_networks_without_launching():
    lib = _lib.load()
    deep = lib.ppo_step_mlp_max_layers() + 1
    assert lib.ppo_step_mlp_categorical_f32(None, 1, 400, 16, 400, deep, None, None, None, 1, 1, 8, None, 6, 1, 1.0,
                                           1, 1, 1) == -1
    assert b"ppo_step_mlp_categorical_f32" in lib.ppo_last_error()
    wide = lib.ppo_step_mlp_max_obs() + 4
    assert lib.ppo_step_mlp_categorical_f32(None, 1, wide, 16, wide, 2, None, None, None, 1, 1, 8, None, 6, 1, 1.0,
                                           1, 1, 1) == -1
    # head wider than 16 outputs
    assert lib.ppo_step_mlp_categorical_f32(None, 1, 400, 16, 400, 2, None, None, None, 1, 1, 20, None, 6, 1, 1.0,
                                           1, 1, 1) == -1


def test_vtrace_rejects_a_short_ratio_pitch_without_launching():
    lib = _lib.load()
    assert lib.ppo_vtrace_f32(None, 1, 1, 1, 1, 1, 1, 3, 1.0, 1.0, 1, 1, 4, 8, 0.99, 0.95, 0) == -1
    assert b"ppo_vtrace_f32" in lib.ppo_last_error()


def test_permutation_buckets_fit_the_lds_sort_at_large_sizes():
    """Up to 2^24 items per epoch the expected bucket (n / 2^bits) plus six
    standard deviations of its Poisson count stays within the LDS sort's
    capacity, so the global-memory ranking is not expected to run."""
    lib = _lib.load()
    for e in range(1, 25):
        for n in ((1 << e) - 1, 1 << e, 3 << (e - 1)):
            bits, cap = lib.ppo_permutation_bucket_bits(n), lib.ppo_permutation_bucket_cap(n)
            mean = n / (1 << bits)
            assert mean + 6 * mean ** 0.5 <= cap or n <= cap, (n, bits, cap)
