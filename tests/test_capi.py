"""The C-ABI library loads, exports every entry point include/lazylora_mxfp4.h declares, and
rejects bad arguments on the host before anything reaches a device. No GPU needed."""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lazylora_mxfp4.h")


@pytest.fixture(scope="module")
def lib():
    from lazylora_amd import native
    if not os.path.exists(native.LIB_PATH):
        pytest.fail(f"{native.LIB_PATH} is not built: run __graft_entry__.build() first")
    return native._load_library()


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mxfp4_\w+)\s*\(", text)))


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 10, names
    for n in names:
        assert hasattr(lib, n), f"{n} declared in the header but not exported"


def test_workspace_queries(lib):
    assert lib.mxfp4_gemm_workspace_size(16, 7168, 2048) >= 2 * 16 * 7168
    assert lib.mxfp4_gemm_t_workspace_size(16, 7168, 2048) >= 2 * 2 * 16 * 2048
    big = lib.mxfp4_moe_workspace_size(1024, 8, 896, 7168, 2048)
    assert 400 << 20 < big < 1 << 30
    assert lib.mxfp4_moe_workspace_size(0, 0, 1, 1, 1) == 0


def test_host_side_argument_errors(lib):
    vp = ctypes.c_void_p
    dummy = vp(256)  # never dereferenced: every call below must fail its checks first
    assert lib.mxfp4_dequant(dummy, dummy, dummy, 33, 4, None) == -1
    assert b"multiple of 32" in lib.mxfp4_last_error()
    assert lib.mxfp4_gemm(dummy, dummy, dummy, dummy, 4, 48, 4, None, 0, None) == -1
    assert lib.mxfp4_gemm(dummy, dummy, dummy, dummy, 4, 64, 4, None, 0, None) == -2
    assert lib.mxfp4_gemm_t(dummy, dummy, dummy, dummy, 4, 64, 4, None, 0, None) == -2
    args = [dummy, dummy, 0, dummy, 3, dummy, 4, 2] + [dummy] * 6 + [8, 64, 32]
    assert lib.mxfp4_moe_forward(*args, 7, 0, dummy, 1 << 40, None) == -1   # unknown activation
    assert lib.mxfp4_moe_forward(*args, 0, 0, dummy, 16, None) == -2        # workspace too small
    bad = [dummy, dummy, 0, dummy, 3, dummy, 4, 2] + [dummy] * 6 + [8, 60, 32]
    assert lib.mxfp4_moe_forward(*bad, 0, 0, dummy, 1 << 40, None) == -1    # D % 32 != 0
    unaligned = [dummy, dummy, 0, dummy, 3, dummy, 4, 2, vp(257)] + [dummy] * 5 + [8, 64, 32]
    assert lib.mxfp4_moe_forward(*unaligned, 0, 0, dummy, 1 << 40, None) == -1
    assert lib.mxfp4_router_topk(dummy, dummy, dummy, None, 4, 100, 65, 1.0, 1, None) == -1  # top_k > 64
    assert b"top_k" in lib.mxfp4_last_error()
    assert lib.mxfp4_router_topk(dummy, dummy, dummy, None, 4, 100, 0, 1.0, 1, None) == -1
    assert lib.mxfp4_router_topk(dummy, dummy, dummy, None, 4, 4097, 8, 1.0, 1, None) == -1  # E > 4096
    assert lib.mxfp4_router_topk(None, dummy, dummy, None, 4, 100, 8, 1.0, 1, None) == -1    # null output
    assert lib.mxfp4_router_topk(None, None, None, None, 0, 100, 8, 1.0, 1, None) == 0       # N = 0: no-op
    assert lib.mxfp4_router_topk_backward(dummy, dummy, dummy, dummy, 4, 8, 9, 1.0, 1, None) == -1


def test_python_api_validation():
    from lazylora_amd.native import kernel
    k = kernel()
    x = torch.zeros(2, 64)
    with pytest.raises(ValueError):
        k.gemm(x, torch.zeros(8, 16, dtype=torch.uint8), torch.zeros(8, 2, dtype=torch.uint8))
    with pytest.raises(ValueError):
        k.gemm(torch.zeros(2, 48), torch.zeros(8, 24, dtype=torch.uint8), torch.zeros(8, 1, dtype=torch.uint8))
    with pytest.raises(ValueError):
        k.gemm_t(torch.zeros(2, 7), torch.zeros(8, 32, dtype=torch.uint8), torch.zeros(8, 2, dtype=torch.uint8))
    with pytest.raises(ValueError):
        k.dequant(torch.zeros(8, 32, dtype=torch.uint8), torch.zeros(8, 3, dtype=torch.uint8))
    from lazylora_amd.experts import ExpertLayer
    z = torch.zeros
    with pytest.raises(ValueError):
        ExpertLayer(z(2, 32, 32, dtype=torch.uint8), z(2, 32, 2, dtype=torch.uint8), z(2, 32, 32, dtype=torch.uint8),
                    z(2, 32, 2, dtype=torch.uint8), z(2, 64, 16, dtype=torch.uint8), z(2, 64, 3, dtype=torch.uint8))


def test_no_native_opt_out(monkeypatch):
    from lazylora_amd import native
    monkeypatch.setenv("LAZYLORA_NO_NATIVE", "1")
    assert native.kernel() is None


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from lazylora_amd import native
    monkeypatch.setattr(native, "_lib", None)
    monkeypatch.setattr(native, "_kernel", None)
    monkeypatch.setattr(native, "LIB_PATH", str(tmp_path / "absent.so"))
    with pytest.raises(RuntimeError, match="missing"):
        native.kernel()
