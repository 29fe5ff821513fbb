"""Host-side checks of the native code (CPU; they need hipcc, not a GPU).

* The SGPR-base DMA address (lds_dma16_sbase): a device address split into
  halves by readfirstlane (which returns int) and joined again must survive
  when the low half has bit 31 set -- the fault of an earlier build, whose
  join sign-extended that half (tests/host/check_dma_base.hip).
* The two query rows of a selection tile (pair_rows): addressed upward from
  the lower query, so a CSR whose entries do not ascend cannot wrap an
  unsigned offset (tests/host/check_pair_rows.hip).
* A row-tile request that starts at or past the end of its source reads the
  last row instead of wrapping an unsigned offset (tile_rows,
  tests/host/check_tile_rows.hip).
* M0: the inline-asm DMA helpers of nsa_tile32.h write M0 (the LDS address
  of global_load_lds) behind the compiler's back.  That is safe only while
  no compiler-generated instruction keeps a value in M0 across them.  The
  device assembly of every kernel file is checked: every M0 write is one of
  the helpers' own ``s_mov_b32 m0`` immediately followed by its
  ``global_load_lds``, and no instruction that reads M0 implicitly (movrel,
  GWS, sendmsg, LDS-returning buffer loads) appears anywhere.
"""

import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "openbox-llm_amd")
HIPCC = "/opt/rocm/bin/hipcc"

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC), reason="needs hipcc")


def test_dma_base_address_halves(tmp_path):
    exe = tmp_path / "check_dma_base"
    subprocess.run([HIPCC, "-std=c++17", "-O1", "--offload-arch=gfx950", f"-I{ROOT}/include", f"-I{PKG}/csrc",
                    os.path.join(ROOT, "tests", "host", "check_dma_base.hip"), "-o", str(exe)],
                   check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    print(r.stdout)
    assert r.returncode == 0, r.stdout


def test_pair_rows_addressing(tmp_path):
    """The two queries of a selection tile are addressed upward from the lower
    one, so a CSR whose entries do not ascend cannot produce a wrapped offset
    (the regression of an out-of-bounds read; tests/host/check_pair_rows.hip)."""
    exe = tmp_path / "check_pair_rows"
    subprocess.run([HIPCC, "-std=c++17", "-O1", "--offload-arch=gfx950", f"-I{ROOT}/include", f"-I{PKG}/csrc",
                    os.path.join(ROOT, "tests", "host", "check_pair_rows.hip"), "-o", str(exe)],
                   check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    print(r.stdout)
    assert r.returncode == 0, r.stdout


def test_tile_rows_clamp(tmp_path):
    """Row-tile requests from any start row, also past the end of the source,
    address only rows of the source (tests/host/check_tile_rows.hip)."""
    exe = tmp_path / "check_tile_rows"
    subprocess.run([HIPCC, "-std=c++17", "-O1", "--offload-arch=gfx950", f"-I{ROOT}/include", f"-I{PKG}/csrc",
                    os.path.join(ROOT, "tests", "host", "check_tile_rows.hip"), "-o", str(exe)],
                   check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    print(r.stdout)
    assert r.returncode == 0, r.stdout


# instructions that read M0 without naming it
IMPLICIT_M0 = re.compile(r"^\s*(s_movrel|v_movrel|ds_gws|ds_append|ds_consume|s_sendmsg|v_interp|s_ttracedata|"
                         r"buffer_load_\w+.*\blds\b)")


def test_m0_is_written_only_by_the_dma_helpers():
    if shutil.which("make") is None:
        pytest.skip("needs make")
    subprocess.run(["make", "-s", "-j8", "-C", PKG, "asm"], check=True, capture_output=True)
    build = os.path.join(PKG, "_build")
    checked = 0
    for name in sorted(os.listdir(build)):
        if not name.endswith(".s"):
            continue
        lines = [ln.strip() for ln in open(os.path.join(build, name))
                 if ln.strip() and not ln.strip().startswith((";", ".", "//"))]
        for i, ln in enumerate(lines):
            assert not IMPLICIT_M0.match(ln), f"{name}: compiler instruction reading M0: {ln}"
            if re.search(r"\bm0\b", ln):
                assert ln.startswith("s_mov_b32 m0,"), f"{name}: M0 used outside the DMA helpers: {ln}"
                nxt = lines[i + 1:i + 3]
                assert nxt[0].startswith("s_nop 0") and nxt[1].startswith("global_load_lds_dword"), \
                    f"{name}: M0 write not followed by its DMA: {ln} / {nxt}"
                checked += 1
            elif ln.startswith("global_load_lds_dword"):
                assert lines[i - 2].startswith("s_mov_b32 m0,"), f"{name}: DMA without its M0 write: {ln}"
    assert checked > 0


def test_flat_row_visibility(tmp_path):
    """The range dK/dV's flat-row masks (groups of G < 16 heads, row R =
    query R / G) against brute force over every row of a tile, window and
    compression (tests/host/check_flat_rows.hip)."""
    exe = tmp_path / "check_flat_rows"
    subprocess.run([HIPCC, "-std=c++17", "-O1", "--offload-arch=gfx950", f"-I{ROOT}/include", f"-I{PKG}/csrc",
                    os.path.join(ROOT, "tests", "host", "check_flat_rows.hip"), "-o", str(exe)],
                   check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    print(r.stdout)
    assert r.returncode == 0, r.stdout
