"""The C-ABI library loads (no GPU needed) and exports every function include/*.h declares."""
import re
from pathlib import Path

from torchinferno_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def declared_functions() -> set[str]:
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(ti_[a-z0-9_]+)\s*\(", text))
    return names


def test_header_declares_entry_points():
    assert {"ti_w4a16_gemm", "ti_int4_repack", "ti_int4_dequant"} <= declared_functions()


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    missing = [n for n in sorted(declared_functions()) if not hasattr(lib, n)]
    assert not missing, missing


def test_python_signatures_cover_header():
    assert declared_functions() == set(_lib.SIGNATURES)


def test_host_side_queries():
    lib = _lib.lib()
    assert lib.ti_version() >= 100
    assert lib.ti_int4_packed_weight_bytes(4096, 4096) == 4096 * 4096 // 2
    # Unsupported shapes report zero workspace and no crash.
    assert lib.ti_w4a16_workspace_bytes(1, 100, 256, 128) == 0
    assert lib.ti_w4a16_workspace_bytes(16, 4096, 14336, 128) > 0  # split-K plan


def test_gemm_rejects_bad_arguments_without_gpu():
    """Argument checks run on the host before any launch."""
    lib = _lib.lib()
    st = lib.ti_w4a16_gemm(None, 2, None, None, None, 1, 64, 128, 128, None, 0, None)
    assert st == _lib.TI_ERR_INVALID
    assert b"null" in lib.ti_last_error()
    st = lib.ti_w4a16_gemm(16, 2, 16, 16, 16, 1, 100, 128, 128, None, 0, None)
    assert st == _lib.TI_ERR_UNSUPPORTED


def test_every_int4_plan_is_launchable(monkeypatch):
    """Host-side plan selection names an instantiated kernel whose workgroups tile N
    exactly, for every M and every N granularity, under the tuning overrides too."""
    import ctypes
    lib = _lib.lib()
    buf = ctypes.create_string_buffer(256)
    cases = [(k, n) for k in (128, 1024, 4096, 14336) for n in (64, 192, 320, 512, 4096, 28672)]
    for mr in (None, "4", "16", "32", "64", "128"):
        for plan in (None, "1:1:3:1", "4:4:6:8", "2:2:2:1", "4:1:2:2"):
            if mr:
                monkeypatch.setenv("TI_ROCM_W4A16_DECODE_MR", mr)
            else:
                monkeypatch.delenv("TI_ROCM_W4A16_DECODE_MR", raising=False)
            if plan:
                monkeypatch.setenv("TI_ROCM_W4A16_DECODE_PLAN", plan)
            else:
                monkeypatch.delenv("TI_ROCM_W4A16_DECODE_PLAN", raising=False)
            monkeypatch.setenv("TI_ROCM_W4A16_DECODE_MIN_M", "1")
            monkeypatch.setenv("TI_ROCM_W4A16_DECODE_MAX_M", "4096")
            for k, n in cases:
                for m in (1, 3, 17, 33, 64, 65, 128, 129, 300):
                    st = lib.ti_w4a16_plan_name(m, n, k, 128, buf, 256)
                    assert st == 0, (mr, plan, m, n, k, lib.ti_last_error())
