"""CPU-side checks of the drop-in boundary: the HIP library loads without a GPU
and exports every function include/*.h declares (no compute calls here)."""
import ctypes
import re

import pytest

from conftest import ROOT


def declared_functions():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(lbh_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("lbh_quantize_row_q8_k_into", "lbh_gemv_into", "lbh_gemv_accumulate_scaled_into",
                 "lbh_matrix_create", "lbh_gemv_q8_k", "lbh_gemv_block_sums", "lbh_backend_name"):
        assert must in names


def test_library_exports_every_declared_symbol():
    import lbhip
    if not lbhip.LIB_PATH.exists():
        pytest.fail(f"{lbhip.LIB_PATH} not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(str(lbhip.LIB_PATH))
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_backend_name_and_device_probe_without_gpu():
    import lbhip
    assert lbhip.backend_name() == "hip_gfx950_q8_k"
    assert lbhip.lib().lbh_device_count() >= 0


def test_oracle_is_not_linked_into_the_product():
    import subprocess
    import lbhip
    out = subprocess.run(["ldd", str(lbhip.LIB_PATH)], capture_output=True, text=True).stdout
    assert "lb_oracle" not in out
    for src in (ROOT / "lightbridge-engine_amd").rglob("*"):
        if src.suffix in (".py", ".hip", ".h", ".cpp") and src.is_file():
            assert "lb_oracle" not in src.read_text(errors="ignore"), src


def test_noalloc_scratch_limit_is_the_documented_token_count():
    """lbh_gemm_q8_k_noalloc admits a batch while lbh_gemm_workspace_bytes(n, k) fits
    LBH_NOALLOC_SCRATCH_BYTES: exactly 928 tokens at k = 4096 and 544 at k = 7168,
    the limits the header states (host arithmetic, no GPU)."""
    import lbhip
    hb = lbhip.HipBackend
    limit = hb.NOALLOC_SCRATCH_BYTES
    text = (ROOT / "include" / "lightbridge_hip.h").read_text()
    assert int(re.search(r"#define LBH_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", text).group(1)) << 20 == limit
    for k, n in ((4096, 928), (7168, 544)):
        assert hb.gemm_workspace_bytes(n, k) <= limit < hb.gemm_workspace_bytes(n + 1, k)
        assert f"{n} tokens at k = {k}" in text
