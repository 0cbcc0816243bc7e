"""The compiled C++ adapter (Kidi's PACKED_LINEAR plug-in over the C ABI, kidi_amd/adapter) on the CPU: the library
loads and exports its surface, operation names follow runtime/operator.cpp:21-61, and prepare routes as the
reference's hooks do: the graph::Compiler interceptor declines every operation but PACKED_LINEAR (compiler.h:37-40),
the backend raises UNSUPPORTED for them (no GPU call is made on these paths)."""

import ctypes
import os

import pytest

from tests import adapter_lib

# runtime/operator.cpp:21-61, in Operation order (operator.h:44-84)
NAMES = ["add", "multiply", "cast", "matmul", "linear", "quantized_linear", "gelu", "layer_norm", "softmax",
         "log_softmax", "transpose", "slice", "gather", "concat", "scatter", "attention", "residual_norm", "rms_norm",
         "tanh", "rotary", "packed_linear", "rms_norm_residual", "static_round", "greedy_token", "rms_rotary",
         "gelu_multiply", "silu_multiply", "silu_gate", "embedding", "gated_feed_forward", "diffusion_candidates",
         "diffusion_update", "embedding_sum", "conv1d", "snake_conv1d", "snake_quantized_linear", "conv_transpose_fold",
         "snake", "gelu_gate"]
PACKED_LINEAR = NAMES.index("packed_linear")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(adapter_lib.PATH):
        pytest.skip("adapter not built")
    return adapter_lib.load()


def test_exports(lib):
    for name in adapter_lib.EXPORTS:
        assert hasattr(lib, name), name


def test_operation_names(lib):
    assert [lib.kqa_operation_name(i).decode() for i in range(len(NAMES))] == NAMES
    assert lib.kqa_operation_name(len(NAMES)) is None


def test_interceptor_declines_other_operations(lib):
    for op in range(len(NAMES)):
        if op != PACKED_LINEAR:
            assert lib.kqa_prepare_other(op, 0) == -1  # nullptr: the backend runs it


def test_backend_rejects_other_operations(lib):
    assert lib.kqa_prepare_other(NAMES.index("rms_norm"), 1) == 4  # UNSUPPORTED
    assert adapter_lib.error() == "operation rms_norm is not supported by the HIP backend"
