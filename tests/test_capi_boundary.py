"""The C-ABI library loads, exports every symbol include/llmr_hip.h declares,
and rejects bad arguments before touching a device. No GPU compute."""
import ctypes

import pytest

from llmr_amd import capi, gguf


def test_library_exports_every_declared_symbol():
    names = capi.header_symbols()
    assert len(names) >= 15
    L = capi.lib()
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    assert set(names) == set(capi._SIGS), "ctypes signatures out of sync with the header"


@pytest.mark.parametrize("t,n", [(gguf.GGML_Q8_0, 3072), (gguf.GGML_Q4_K, 15360),
                                 (gguf.GGML_F32, 7), (gguf.GGML_BF16, 9), (gguf.GGML_F16, 1)])
def test_row_bytes_matches_gguf_sizes(t, n):
    assert capi.lib().llmr_ggml_row_bytes(t, n) == gguf.row_bytes(t, n)


def test_row_bytes_rejects_partial_blocks_and_unknown_types():
    L = capi.lib()
    assert L.llmr_ggml_row_bytes(gguf.GGML_Q8_0, 48) == 0
    assert L.llmr_ggml_row_bytes(gguf.GGML_Q4_K, 512 + 32) == 0
    assert L.llmr_ggml_row_bytes(14, 256) == 0  # Q6_K: not implemented here


def test_null_context_is_rejected():
    L = capi.lib()
    rc = L.llmr_batch_matmul(None, 16, 8, 16, 0, 16, 64, 64, 1, 0)
    assert rc == capi.LLMR_ERR_INVALID_ARG
    assert "context" in capi.last_error()
    rc = L.llmr_flash_attention(None, 16, 16, 16, 1, 16, 128, 1, 1, ctypes.c_float(0.1))
    assert rc == capi.LLMR_ERR_INVALID_ARG
    rc = L.llmr_sync(None)
    assert rc == capi.LLMR_ERR_INVALID_ARG
    rc = L.llmr_batch_matmul_pc(None, 16, 8, 16, 0, 16, None)
    assert rc == capi.LLMR_ERR_INVALID_ARG


def test_create_context_without_device_fails_cleanly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a device is present")
    h = ctypes.c_void_p()
    rc = capi.lib().llmr_create_context(0, ctypes.byref(h))
    assert rc == capi.LLMR_ERR_NO_DEVICE and not h
    assert capi.lib().llmr_create_context(0, None) == capi.LLMR_ERR_INVALID_ARG


def _c_harness(name: str) -> str:
    """tests/c/_build/<name>, (re)built with gcc from tests/c when it is
    missing or older than its source, the header or the library."""
    import os
    import subprocess
    cdir = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c")
    exe = os.path.join(cdir, "_build", name)
    subprocess.run(["make", "-C", cdir, f"_build/{name}"], check=True, capture_output=True)
    return exe


def test_header_compiles_as_c11_and_every_entry_point_links():
    """tests/c/abi_symbols.c includes the header under gcc -std=c11 -pedantic
    -Werror and references every declared entry point; it links against the
    library and runs (loading it, touching no device)."""
    import os
    import re
    import subprocess
    exe = _c_harness("abi_symbols")
    src = open(os.path.join(os.path.dirname(exe), "..", "abi_symbols.c")).read()
    listed = re.findall(r'\{"(llmr_\w+)", ', src)
    assert sorted(listed) == sorted(capi.header_symbols()), "abi_symbols.c out of sync with the header"
    out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    n = len(listed)
    assert out.strip() == f"{n} of {n} entry points resolved"


def test_gemm_planner_sweep():
    """tests/c/plan_check.cpp runs the GEMM dispatcher's planner
    (llm-runner_amd/csrc/gemm_plan.h, host-only) over a grid of shapes, CU
    counts and workspace limits: every split launch gives each split at least
    one K stage (the kernels load a split's first stage unconditionally; M
    320 x N 640 x K 3072 on 256 CUs once had an empty eleventh split), every
    plan stays within its workspace limit, and f32 activations are rounded to
    fp16 against Q8_0 and to bf16 against Q4_K."""
    import subprocess
    exe = _c_harness("plan_check")
    out = subprocess.run([exe], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.startswith("plan_check: ") and out.stdout.strip().endswith("plans ok")
