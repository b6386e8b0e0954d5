"""The C++ host API (higgs_amd/host/higgs.hpp, built into higgs_amd/libhiggs.so)
and its parity program tests/cpp/test_host_api.cpp, which checks each
layer-level call against the oracle on the GPU."""
from __future__ import annotations

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "_build", "test_host_api")
HOST_LIB = os.path.join(ROOT, "higgs_amd", "libhiggs.so")

EXPECTED = {
    "test_swiglu", "test_swiglu_numeric_correctness", "test_from_slice_rounds_like_the_oracle",
    "test_views_read_back_in_logical_order", "test_rms_norm_matches_oracle_bf16",
    "test_rms_norm_gemma_plus_one_is_float32", "test_rms_norm_strided_rows_f16",
    "test_apply_rope_default_bf16", "test_apply_rope_llama3_freqs",
    "test_apply_rope_partial_passes_tail_through",
    "test_apply_rope_batched_equals_per_request_loop", "test_qk_norm_rope_matches_oracle",
    "test_gated_rms_norm_reads_z_in_place", "test_silu_mul_and_gelu_approximate_mul",
    "test_swiglu_fused_gate_up_halves", "test_quantized_embedding_llama_table",
    "test_empty_inputs_give_empty_results", "test_errors_name_the_op_and_operands",
    "test_ops_run_on_the_scoped_stream", "test_add_rms_norm_block_boundaries",
    "test_quantized_embedding_forward_rms_norm",
    "test_load_quantized_checkpoint_drives_embedding_and_norm", "test_switch_mlp_forward_gather",
    "test_gated_delta_reference_cases_and_decode", "test_qlinear_forward_matches_oracle",
    "test_array_outlives_its_stream_and_orders_cross_stream_frees",
}


def _need_exe():
    if not os.path.exists(EXE):
        pytest.fail("tests/cpp/_build/test_host_api is missing: run __graft_entry__.build()")


def test_cpp_parity_program_lists_every_case():
    _need_exe()
    r = subprocess.run([EXE, "--list"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    assert set(r.stdout.split()) == EXPECTED


def test_host_library_exports_the_mlx_shaped_api():
    if not os.path.exists(HOST_LIB):
        pytest.fail("higgs_amd/libhiggs.so is missing: run __graft_entry__.build()")
    out = subprocess.run(["nm", "-DC", "--defined-only", HOST_LIB], capture_output=True,
                         text=True, check=True).stdout
    for sym in ("higgs::fast::rms_norm(", "higgs::fast::rope(", "higgs::fast::rope_batched(",
                "higgs::nn::RmsNorm::forward(", "higgs::nn::Rope::forward(",
                "higgs::nn::QuantizedEmbedding::forward(", "higgs::nn::silu_mul(",
                "higgs::nn::gelu_approximate_mul(", "higgs::apply_rope(", "higgs::swiglu(",
                "higgs::gated_delta(", "higgs::gdn_qk_norm_weights(", "higgs::quantized_matmul(",
                "higgs::nn::QLinear::forward(",
                "higgs::gated_rms_norm(", "higgs::qk_norm_rope(", "higgs::Array::from_slice(",
                "higgs::add_rms_norm(", "higgs::nn::QuantizedEmbedding::forward_rms_norm(",
                "higgs::gather_qmm(", "higgs::nn::SwitchMlpWeights::forward_gather("):
        assert sym in out, sym
    # the host library reaches the kernels only through the C ABI
    dyn = subprocess.run(["nm", "-D", "--undefined-only", HOST_LIB], capture_output=True,
                         text=True, check=True).stdout
    for fn in ("hgk_rms_norm", "hgk_rope", "hgk_qk_norm_rope", "hgk_glu", "hgk_gated_rms_norm",
               "hgk_quantized_embedding", "hgk_last_error", "hgk_add_rms_norm",
               "hgk_quantized_embedding_rms_norm", "hgk_gather_qmm", "hgk_quantized_matmul",
               "hgk_gated_delta", "hgk_sync"):
        assert fn in dyn, fn


@pytest.mark.gpu
def test_cpp_host_api_parity_on_gpu():
    _need_exe()
    print("[cpp] running tests/cpp/_build/test_host_api", flush=True)
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=300)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert f"{len(EXPECTED)} run, 0 failed" in r.stdout
