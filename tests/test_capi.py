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
    assert lib.mxfp4_dequant_bf16(dummy, dummy, dummy, 33, 4, None) == -1
    assert lib.mxfp4_dequant_bf16(None, dummy, dummy, 64, 4, None) == -1      # null output
    assert lib.mxfp4_dequant_bf16(None, None, None, 64, 0, None) == 0         # R = 0: no-op
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


def test_forward_layout_host_checks(lib):
    vp = ctypes.c_void_p
    dummy = vp(256)  # never dereferenced: every call below fails (or finishes) before a launch
    # 2 experts x 3 row groups (R = 40: the last group holds 8 rows) x 2 super-chunks x (4 KiB of
    # codes + 256 B of scales)
    assert lib.mxfp4_forward_layout_bytes(2, 40, 1024) == 2 * 3 * 2 * (4096 + 256)
    assert lib.mxfp4_forward_layout_bytes(2, 40, 1056) == 0  # K not a multiple of 512
    far = vp(1 << 40)  # scales far from every other range below
    assert lib.mxfp4_forward_layout(dummy, dummy, far, 2, 40, 1056, None) == -1
    assert b"multiple of 512" in lib.mxfp4_last_error()
    assert lib.mxfp4_forward_layout(None, dummy, far, 2, 40, 1024, None) == -1     # null output
    assert lib.mxfp4_forward_layout(dummy, dummy, None, 2, 40, 1024, None) == -1   # null scales
    assert lib.mxfp4_forward_layout(vp(264), dummy, far, 2, 40, 1024, None) == -1  # unaligned output
    assert lib.mxfp4_forward_layout(dummy, vp(1 << 41), vp(264), 2, 40, 1024, None) == -1  # unaligned scales
    assert lib.mxfp4_forward_layout(dummy, vp(256 + 4096), far, 2, 40, 1024, None) == -1  # overlapping codes
    assert b"overlaps" in lib.mxfp4_last_error()
    assert lib.mxfp4_forward_layout(dummy, vp(1 << 41), vp(256 + 4096), 2, 40, 1024, None) == -1  # overlapping scales
    assert b"overlaps" in lib.mxfp4_last_error()
    assert lib.mxfp4_forward_layout(None, None, None, 0, 40, 1024, None) == 0       # E = 0: no-op
    # the routed calls with forward layouts {W1, W3, W2}: D = 1024, F = 544
    args = [dummy, dummy, 0, dummy, 3, dummy, 4, 2] + [dummy] * 6
    tail = [8, 1024, 544, 0, None, None, 0, 0, dummy, 1 << 40, None]
    fl_w2 = (vp * 3)(None, None, 256)      # W2's K = F = 544 is not a multiple of 512
    assert lib.mxfp4_moe_forward_fl(*args, fl_w2, *tail) == -1
    assert b"multiple of 512" in lib.mxfp4_last_error()
    fl_w1 = (vp * 3)(256, None, None)      # W1 without W3
    assert lib.mxfp4_moe_forward_fl(*args, fl_w1, *tail) == -1
    assert b"together" in lib.mxfp4_last_error()
    fl_odd = (vp * 3)(256, 264, None)      # unaligned
    assert lib.mxfp4_moe_forward_fl(*args, fl_odd, *tail) == -1
    btail = [8, 1024, 544, 0, None, None, 0, None, 0, dummy, 1 << 40, None]
    assert lib.mxfp4_moe_backward_fl(dummy, dummy, dummy, dummy, 0, dummy, 3, dummy, 4, 2, *([dummy] * 6),
                                     fl_w1, *btail) == -1
    # without tokens the forward has nothing to do: valid layouts and no launch
    ok = (vp * 3)(256, 512, None)
    tail0 = [8, 1024, 544, 0, None, None, 0, 0, dummy, 1 << 40, None]
    assert lib.mxfp4_moe_forward_fl(dummy, dummy, 0, dummy, 3, dummy, 0, 2, *([dummy] * 6), ok, *tail0) == 0


def test_backward_layout_host_checks(lib):
    vp = ctypes.c_void_p
    dummy = vp(256)  # never dereferenced: every call below fails (or finishes) before a launch
    # per expert R * (K/2 + K/32): the codes and scales, rearranged into (32-row step, 256-column
    # stripe) blocks
    assert lib.mxfp4_backward_layout_bytes(2, 64, 512) == 2 * 64 * (256 + 16)
    assert lib.mxfp4_backward_layout_bytes(2, 40, 512) == 0  # R not a multiple of 32
    assert lib.mxfp4_backward_layout_bytes(2, 64, 384) == 0  # K not a multiple of 256
    far = vp(1 << 40)
    assert lib.mxfp4_backward_layout(dummy, dummy, far, 2, 64, 384, None) == -1
    assert b"K of 256" in lib.mxfp4_last_error()
    assert lib.mxfp4_backward_layout(dummy, dummy, far, 2, 40, 512, None) == -1
    assert lib.mxfp4_backward_layout(None, dummy, far, 2, 64, 512, None) == -1     # null output
    assert lib.mxfp4_backward_layout(dummy, dummy, None, 2, 64, 512, None) == -1   # null scales
    assert lib.mxfp4_backward_layout(vp(264), dummy, far, 2, 64, 512, None) == -1  # unaligned output
    assert lib.mxfp4_backward_layout(dummy, vp(256 + 4096), far, 2, 64, 512, None) == -1  # overlapping codes
    assert b"overlaps" in lib.mxfp4_last_error()
    assert lib.mxfp4_backward_layout(dummy, vp(1 << 41), vp(256 + 4096), 2, 64, 512, None) == -1
    assert b"overlaps" in lib.mxfp4_last_error()
    assert lib.mxfp4_backward_layout(None, None, None, 0, 64, 512, None) == 0       # E = 0: no-op
    # the routed calls with MXFP4_MOE_BWD_LAYOUT read six entries: D = 1024, F = 544
    args = [dummy, dummy, 0, dummy, 3, dummy, 4, 2] + [dummy] * 6
    tail = [8, 1024, 544, 0, None, None, 0, 4, dummy, 1 << 40, None]
    bl_w2 = (vp * 6)(None, None, None, None, None, 256)  # W2's K = F = 544 is not a multiple of 256
    assert lib.mxfp4_moe_forward_fl(*args, bl_w2, *tail) == -1
    assert b"multiple of 256" in lib.mxfp4_last_error()
    bl_w1 = (vp * 6)(None, None, None, 256, None, None)  # W1 without W3
    assert lib.mxfp4_moe_forward_fl(*args, bl_w1, *tail) == -1
    assert b"together" in lib.mxfp4_last_error()
    bl_odd = (vp * 6)(None, None, None, 256, 264, None)  # unaligned
    assert lib.mxfp4_moe_forward_fl(*args, bl_odd, *tail) == -1
    btail = [8, 1024, 544, 0, None, None, 0, None, 4, dummy, 1 << 40, None]
    assert lib.mxfp4_moe_backward_fl(dummy, dummy, dummy, dummy, 0, dummy, 3, dummy, 4, 2, *([dummy] * 6),
                                     bl_w1, *btail) == -1
    # without the flag only the first three entries are read: the same array passes
    tail_noflag = [8, 1024, 544, 0, None, None, 0, 0, dummy, 1 << 40, None]
    assert lib.mxfp4_moe_forward_fl(dummy, dummy, 0, dummy, 3, dummy, 0, 2, *([dummy] * 6), bl_w2,
                                    *tail_noflag) == 0
    ok = (vp * 6)(256, 512, None, 768, 1024, None)
    assert lib.mxfp4_moe_forward_fl(dummy, dummy, 0, dummy, 3, dummy, 0, 2, *([dummy] * 6), ok, *tail) == 0


def test_python_api_validation(lib):
    from lazylora_amd import native
    k = native.MXFP4Kernel(lib)  # the shape checks run before any device is needed
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


def _fresh(monkeypatch, native):
    monkeypatch.setattr(native, "_lib", None)
    monkeypatch.setattr(native, "_kernel", None)
    monkeypatch.setattr(native, "_tried", False)
    monkeypatch.delenv("LAZYLORA_NO_NATIVE", raising=False)
    monkeypatch.delenv("LAZYLORA_NATIVE_STRICT", raising=False)


def test_missing_library_gives_none(monkeypatch, tmp_path, capsys):
    """The reference's contract (native/__init__.py:77-96): an unavailable library is None plus a
    warning, so a caller that probes `kernel() is not None` (expert_streamer.py:206-207) falls
    back instead of crashing."""
    from lazylora_amd import native
    _fresh(monkeypatch, native)
    monkeypatch.setattr(native, "LIB_PATH", str(tmp_path / "absent.so"))
    assert native.kernel() is None
    assert "not available" in capsys.readouterr().err
    assert native.kernel() is None  # the failed attempt is not repeated
    keep_packed = native.kernel() is not None  # the streamer's probe
    assert keep_packed is False


def test_unloadable_library_gives_none(monkeypatch, tmp_path):
    from lazylora_amd import native
    _fresh(monkeypatch, native)
    bad = tmp_path / "broken.so"
    bad.write_bytes(b"not an ELF file")
    monkeypatch.setattr(native, "LIB_PATH", str(bad))
    assert native.kernel() is None


def test_strict_mode_raises(monkeypatch, tmp_path):
    from lazylora_amd import native
    _fresh(monkeypatch, native)
    monkeypatch.setattr(native, "LIB_PATH", str(tmp_path / "absent.so"))
    monkeypatch.setenv("LAZYLORA_NATIVE_STRICT", "1")
    with pytest.raises(RuntimeError, match="missing"):
        native.kernel()


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-device case")
def test_no_device_gives_none(monkeypatch):
    from lazylora_amd import native
    _fresh(monkeypatch, native)
    assert native.kernel() is None


def test_alignment_rejected_on_host(lib):
    """Packed weights and scales need 16-byte alignment, gemm's x 8 bytes, gemm_t's dy 4 bytes,
    dequant_bf16's out 4 bytes and the routed layer's h 8 bytes (fp32) / 4 bytes (bf16);
    violations return EINVAL before any launch (include/lazylora_mxfp4.h)."""
    vp = ctypes.c_void_p
    ok, odd8, odd4, odd1 = vp(4096), vp(4096 + 8), vp(4096 + 4), vp(4096 + 1)
    ws = vp(1 << 20)
    assert lib.mxfp4_gemm(ok, ok, ok, odd8, 4, 64, 4, ws, 1 << 30, None) == -1      # scales
    assert b"16-byte" in lib.mxfp4_last_error()
    assert lib.mxfp4_gemm(ok, odd4, ok, ok, 4, 64, 4, ws, 1 << 30, None) == -1      # x
    assert lib.mxfp4_dequant_bf16(vp(4096 + 2), ok, ok, 64, 4, None) == -1         # bf16 out at 2 bytes
    assert b"4-byte" in lib.mxfp4_last_error()
    assert lib.mxfp4_gemm_t(ok, ok, ok, odd8, 4, 64, 4, ws, 1 << 30, None) == -1    # scales
    assert lib.mxfp4_gemm_t(ok, odd1, ok, ok, 4, 64, 4, ws, 1 << 30, None) == -1    # dy
    wts = [ok] * 6
    for i in range(6):  # every packed and scale array of the experts
        w = list(wts)
        w[i] = odd8
        args = [ok, ok, 0, ok, 3, ok, 4, 2] + w + [8, 64, 32]
        assert lib.mxfp4_moe_forward(*args, 0, 0, ws, 1 << 40, None) == -1, i
    args = [ok, odd4, 0, ok, 3, ok, 4, 2] + wts + [8, 64, 32]                   # fp32 h at 4 bytes
    assert lib.mxfp4_moe_forward(*args, 0, 0, ws, 1 << 40, None) == -1
    assert b"h must be" in lib.mxfp4_last_error()
    args = [ok, odd1, 1, ok, 3, ok, 4, 2] + wts + [8, 64, 32]                   # bf16 h at 1 byte
    assert lib.mxfp4_moe_forward(*args, 0, 0, ws, 1 << 40, None) == -1


def test_from_bundles_places_streamed_experts_by_id():
    """ExpertLayer.from_bundles takes the reference's ExpertWeightBundle objects, either as a
    list (expert e at position e) or as the (expert_id, bundle) pairs stream_experts yields in
    disk order (expert_streamer.py:315-369); absent experts are zeros."""
    from types import SimpleNamespace
    from lazylora_amd.experts import ExpertLayer
    D, F = 64, 32
    g = torch.Generator().manual_seed(0)

    def bundle(e):
        def r(*shape):
            return torch.randint(0, 256, shape, generator=g, dtype=torch.uint8)
        return SimpleNamespace(expert_idx=e, packed=True,
                               gate_packed=r(F, D // 2), gate_scale=r(F, D // 32), up_packed=r(F, D // 2),
                               up_scale=r(F, D // 32), down_packed=r(D, F // 2), down_scale=r(D, F // 32))

    streamed = [(5, bundle(5)), (1, bundle(1)), (3, bundle(3))]  # disk order, not id order
    layer = ExpertLayer.from_bundles(streamed, device="cpu", num_experts=8)
    assert (layer.E, layer.D, layer.F) == (8, D, F)
    for eid, b in streamed:
        assert torch.equal(layer.w1p[eid], b.gate_packed) and torch.equal(layer.w1s[eid], b.gate_scale)
        assert torch.equal(layer.w3p[eid], b.up_packed) and torch.equal(layer.w3s[eid], b.up_scale)
        assert torch.equal(layer.w2p[eid], b.down_packed) and torch.equal(layer.w2s[eid], b.down_scale)
    for eid in (0, 2, 4, 6, 7):
        assert int(layer.w1p[eid].abs().sum()) == 0 and int(layer.w2s[eid].abs().sum()) == 0
    listed = ExpertLayer.from_bundles([b for _, b in sorted(streamed)], device="cpu")
    assert listed.E == 3 and torch.equal(listed.w2p[2], streamed[0][1].down_packed)
    with pytest.raises(ValueError):
        ExpertLayer.from_bundles([(2, bundle(2)), (2, bundle(2))], device="cpu")
    with pytest.raises(ValueError):
        ExpertLayer.from_bundles(streamed, device="cpu", num_experts=4)
    unpacked = SimpleNamespace(packed=False, gate_packed=None)
    with pytest.raises(ValueError):
        ExpertLayer.from_bundles([unpacked], device="cpu")


def test_forward_layout_dropped_after_inplace_write():
    """A forward-layout copy made before an in-place write to the codes or scales is stale: the
    layer drops it (with a warning) instead of handing its pointers to the routed calls."""
    import warnings
    from lazylora_amd.experts import ExpertLayer
    E, D, F = 2, 512, 512
    z = lambda *shape: torch.zeros(shape, dtype=torch.uint8)
    L = ExpertLayer(z(E, F, D // 2), z(E, F, D // 32), z(E, F, D // 2), z(E, F, D // 32), z(E, D, F // 2),
                    z(E, D, F // 32), device=torch.device("cpu"))
    assert L.forward_layout_pointers() is None
    L._fl = (z(16), z(16), None)  # stand-ins for the copies prepare_forward_layout makes on a GPU
    L._fl_versions = L._code_versions()
    assert L.forward_layout_pointers() is not None
    L.w2p[1].fill_(3)  # through a view
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        assert L.forward_layout_pointers() is None
    assert any(issubclass(w.category, RuntimeWarning) for w in caught)
    assert L._fl is None
    L._fl = (z(16), z(16), None)  # the copies hold the scales too: a write to them also makes them stale
    L._fl_versions = L._code_versions()
    L.w1s.add_(1)
    with warnings.catch_warnings(record=True):
        warnings.simplefilter("always")
        assert L.forward_layout_pointers() is None


def test_layout_pointers_and_stale_backward_layout():
    """layout_pointers: three forward-layout entries without flags, six entries (forward, then
    backward) with MXFP4_MOE_BWD_LAYOUT once a backward layout exists; a write to the weights
    drops both copies."""
    import warnings
    from lazylora_amd.experts import ExpertLayer
    from lazylora_amd.native import MOE_BWD_LAYOUT
    E, D, F = 2, 512, 512
    z = lambda *shape: torch.zeros(shape, dtype=torch.uint8)
    L = ExpertLayer(z(E, F, D // 2), z(E, F, D // 32), z(E, F, D // 2), z(E, F, D // 32), z(E, D, F // 2),
                    z(E, D, F // 32), device=torch.device("cpu"))
    assert L.layout_pointers() == (None, 0)
    L._fl = (z(16), z(16), None)
    L._fl_versions = L._code_versions()
    arr, flags = L.layout_pointers()
    assert flags == 0 and len(arr) == 3 and arr[2] is None
    L._bl = (z(16), z(16), z(16))
    L._bl_versions = L._code_versions()
    arr, flags = L.layout_pointers()
    assert flags == MOE_BWD_LAYOUT and len(arr) == 6 and arr[0] == L._fl[0].data_ptr()
    assert arr[3] == L._bl[0].data_ptr() and arr[5] == L._bl[2].data_ptr()
    L.drop_forward_layout()
    arr, flags = L.layout_pointers()
    assert flags == MOE_BWD_LAYOUT and arr[0] is None and arr[4] == L._bl[1].data_ptr()
    L.w3p.add_(1)
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        assert L.layout_pointers() == (None, 0)
    assert any(issubclass(w.category, RuntimeWarning) for w in caught)
    assert L._bl is None

