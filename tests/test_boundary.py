"""C-ABI boundary and front contracts (CPU only: no kernel is launched).

Mirrors the CPU-runnable contract classes of the reference's native-front
tests (tests/cuda/test_dense_cuda.py:36-64, test_core_cuda.py:21-52,
test_think_cuda.py:35-68, test_moe_cuda.py:23-42, tests/model/test_cuda_scan.py:
34-68): invalid inputs are rejected before any native call, CPU tensors never
run on a fallback, and error messages keep the reference substrings.
"""

from __future__ import annotations

import ctypes
import json
import re
from pathlib import Path

import pytest
import torch

from koemi_amd import _native
from koemi_amd import core, cuda_scan, dense, loader, moe, think

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "koemi_hip.h"
GOLDEN = json.loads((Path(__file__).parent / "golden" / "kats.json").read_text())
GPU = torch.cuda.is_available()


def declared_symbols() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\**\s+\**(koemi_[a-z0-9_]+)\s*\(", text, flags=re.M))


def test_library_is_built_and_exports_every_declared_symbol():
    symbols = declared_symbols()
    assert len(symbols) >= 20
    assert symbols == set(_native.EXPORTED_SYMBOLS), symbols ^ set(_native.EXPORTED_SYMBOLS)
    handle = ctypes.CDLL(_native.library_path())
    for name in sorted(symbols):
        assert hasattr(handle, name), name
    assert _native.load_library().koemi_abi_version() == 1


def test_library_binds_to_the_hip_runtime_torch_uses():
    _native.load_library()
    maps = Path("/proc/self/maps").read_text().splitlines()
    runtimes = {line.split()[-1] for line in maps if "libamdhip64" in line}
    assert len(runtimes) == 1, runtimes


def test_status_codes_and_last_error_without_launching():
    lib = _native.load_library()
    status = lib.koemi_affine_scan_forward(None, None, None, None, 1, 2, 3, 0, 99, None)
    assert status == _native.ERR_UNSUPPORTED
    assert b"dtype" in lib.koemi_last_error()
    status = lib.koemi_moe_route_hash(None, None, None, _native.I64, None, None, 4, 2, 3, None)
    assert status == _native.ERR_INVALID
    with pytest.raises(_native.NativeCallError, match="koemi_rmsnorm_silu_forward"):
        _native.call("koemi_rmsnorm_silu_forward", None, None, None, None, 1, 0, 1e-6, _native.F32, None)


def test_workspace_queries():
    assert _native.query("koemi_rmsnorm_silu_backward_workspace_bytes", 4096, 512) >= 512 * 4
    assert _native.query("koemi_moe_permute_workspace_bytes", 32768, 2, 16) >= 65536 * 8
    assert _native.query("koemi_moe_grouped_mlp_workspace_bytes", 65536, 1024, 2816, 16, _native.BF16) >= 65536 * 2816 * 2
    assert _native.query("koemi_moe_combine_workspace_bytes", 32768, 2) >= 32768 * 2 * 8


def test_grouped_mlp_rejects_shapes_past_its_limits_before_launching():
    # The pointers are never dereferenced: both shapes fail the entry point's
    # checks before any kernel is launched.
    lib = _native.load_library()
    fake = ctypes.c_void_p(1 << 20)

    def run(width: int, hidden: int, experts: int) -> int:
        need = _native.query("koemi_moe_grouped_mlp_workspace_bytes", 256, width, hidden, experts, _native.BF16)
        return lib.koemi_moe_grouped_mlp(fake, fake, fake, fake, fake, fake, fake, fake, fake, fake,
                                         256, width, hidden, experts, _native.BF16, fake, need, None)

    assert run(65536, 32768, 4) == _native.ERR_UNSUPPORTED  # 32-bit tile offsets
    assert b"2^31" in lib.koemi_last_error()
    assert run(1024, 2816, 9000) == _native.ERR_UNSUPPORTED  # LDS-resident tile prefixes
    assert b"experts" in lib.koemi_last_error()


# -------------------------------------------------------------------- dense


def test_dense_cpu_input_is_rejected_without_fallback():
    r, i = torch.ones((1, 2, 4)), torch.ones((1, 2, 4))
    if GPU:
        with pytest.raises(dense.DenseCudaValidationError, match="must be on CUDA"):
            dense.dense_affine_scan(r, i)
    else:
        with pytest.raises(dense.DenseCudaUnavailableError, match="torch.cuda.is_available"):
            dense.dense_affine_scan(r, i)


def test_dense_invalid_shapes_are_rejected_before_native_calls():
    with pytest.raises(dense.DenseCudaValidationError, match="broadcast"):
        dense.dense_affine_scan(torch.ones((1, 2, 4)), torch.ones((1, 2, 5)))
    with pytest.raises(dense.DenseCudaValidationError, match="initial must have shape"):
        dense.dense_affine_scan(torch.ones((1, 2, 4)), torch.ones((1, 2, 4)), torch.ones((1, 5)))
    with pytest.raises(dense.DenseCudaValidationError, match="same dtype"):
        dense.dense_affine_scan(torch.ones((1, 2, 4)), torch.ones((1, 2, 4), dtype=torch.float64))
    with pytest.raises(dense.DenseCudaValidationError, match="unsupported"):
        dense.dense_affine_scan(torch.ones((1, 2, 4), dtype=torch.int32), torch.ones((1, 2, 4), dtype=torch.int32))


def test_reduce_to_shape_known_answer():
    kat = GOLDEN["reduce_to_shape"]
    reduced = dense._reduce_to_shape(torch.ones(kat["gradient_shape"]), torch.Size(kat["target_shape"]))
    assert torch.equal(reduced, torch.full(kat["target_shape"], kat["expected_value"]))


def test_native_available_reflects_gpu_and_library():
    assert dense.native_cuda_available() == bool(GPU and torch.version.hip and _native.library_built())


# ---------------------------------------------------------------- cuda_scan


def test_cuda_scan_contracts():
    if GPU:
        with pytest.raises(cuda_scan.CudaScanValidationError, match="all scan tensors must be on CUDA"):
            cuda_scan.cuda_affine_scan(torch.ones(1, 2, 3), torch.ones(1, 2, 3))
    else:
        with pytest.raises(cuda_scan.CudaScanUnavailableError, match=r"torch.cuda.is_available\(\) is False"):
            cuda_scan.cuda_affine_scan(torch.ones(1, 2, 3), torch.ones(1, 2, 3))
    with pytest.raises(cuda_scan.CudaScanValidationError, match="same batch and sequence dimensions"):
        cuda_scan.cuda_affine_scan(torch.ones(1, 2, 3), torch.ones(1, 3, 3))
    with pytest.raises(cuda_scan.CudaScanValidationError, match="same dtype"):
        cuda_scan.cuda_affine_scan(torch.ones(1, 2, 3), torch.ones(1, 2, 3, dtype=torch.float64))
    with pytest.raises(cuda_scan.CudaScanValidationError, match="positive integer"):
        cuda_scan.cuda_affine_scan(torch.ones(1, 2, 3), torch.ones(1, 2, 3), chunk_size=0)
    with pytest.raises(cuda_scan.CudaScanValidationError, match="initial must have shape"):
        cuda_scan.cuda_affine_scan(torch.ones(1, 2, 3), torch.ones(1, 2, 3), torch.ones(1, 2))


# --------------------------------------------------------------------- core


def test_core_toolchain_status_and_cpu_rejection():
    status = loader.detect_cuda_toolchain()
    assert isinstance(status.ready, bool) and status.reason
    assert status.ready == loader.cuda_extension_available()
    with pytest.raises(loader.CudaExtensionValidationError):
        core.fused_rmsnorm_silu(torch.ones((2, 8)), torch.ones((8,)))


def test_core_shape_dtype_and_contiguity_contracts():
    with pytest.raises(loader.CudaExtensionValidationError, match="hidden dimension"):
        core.fused_rmsnorm_silu(torch.ones((2, 0)), torch.ones((0,)))
    with pytest.raises(loader.CudaExtensionValidationError, match="same dtype"):
        core.fused_rmsnorm_silu(torch.ones((2, 8)), torch.ones((8,), dtype=torch.float16))
    with pytest.raises(loader.CudaExtensionValidationError, match="must have shape"):
        core.fused_rmsnorm_silu(torch.ones((2, 8)), torch.ones((7,)))
    with pytest.raises(loader.CudaExtensionValidationError, match=r"must have shape \[rows, hidden\]"):
        core.fused_rmsnorm_silu(torch.ones((2, 8, 1)), torch.ones((8,)))


# -------------------------------------------------------------------- think


def _think_cpu_inputs():
    return (torch.randn(2, 5, 8), torch.randn(17, 8), torch.randn(17), torch.randint(0, 17, (2, 5)), torch.ones(2, 5, dtype=torch.bool))


def test_think_cpu_execution_reports_without_fallback():
    inputs = _think_cpu_inputs()
    if GPU:
        with pytest.raises(think.CudaThinkValidationError, match="all think tensors must be on CUDA"):
            think.causal_surprise(*inputs)
    else:
        with pytest.raises(think.CudaThinkUnavailableError, match=r"torch.cuda.is_available\(\) is False"):
            think.causal_surprise(*inputs)


def test_think_contracts_are_rejected_before_dispatch():
    p, w, b, t, v = _think_cpu_inputs()
    with pytest.raises(think.CudaThinkValidationError, match="target_ids and valid_mask"):
        think.causal_surprise(p, w, b, t[:, :-1], v)
    with pytest.raises(think.CudaThinkValidationError, match="share a dtype"):
        think.causal_surprise(p, w.double(), b.double(), t, v)
    with pytest.raises(think.CudaThinkValidationError, match="target_ids must use torch.int64"):
        think.causal_surprise(p, w, b, t.int(), v)
    with pytest.raises(think.CudaThinkValidationError, match="non-negative integer"):
        think.benchmark_causal_surprise(p, w, b, t, v, warmup_iterations=-1)
    with pytest.raises(think.CudaThinkValidationError, match="positive integer"):
        think.benchmark_causal_surprise(p, w, b, t, v, measured_iterations=0)
    with pytest.raises(think.CudaThinkValidationError, match="exactly one"):
        think.salience_admission(torch.rand(4), torch.ones(4, dtype=torch.bool))


# ---------------------------------------------------------------------- moe


def test_moe_cpu_inputs_are_rejected_without_fallback():
    tok = torch.tensor([[1, 2]])
    with pytest.raises(moe.CudaMoeValidationError, match="must be a CUDA tensor"):
        moe.route_topk_valid(tok, torch.tensor([[0, 1]]), torch.ones_like(tok, dtype=torch.bool), expert_count=4, top_k=2)
    with pytest.raises(moe.CudaMoeValidationError, match="must be a CUDA tensor"):
        moe.permute_topk(torch.ones((2, 4)), torch.tensor([[0, 1], [1, 0]]), torch.ones(2, dtype=torch.bool), expert_count=2)


def test_moe_extension_load_reports_unavailable_without_gpu():
    if GPU:
        pytest.skip("a GPU is present; covered by the GPU suite")
    with pytest.raises(moe.CudaMoeUnavailableError, match="torch.cuda.is_available"):
        moe.load_native_extension()
