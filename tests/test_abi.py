"""The C ABI library: loads, exports every declared symbol, validates
arguments before touching the GPU.  Runs without a GPU."""
import ctypes
import os
import subprocess
import sys

import pytest

import hipgemm_amd as hg

INVALID = 1  # hipErrorInvalidValue
FAKE = 1 << 20  # aligned fake device address; never dereferenced here


def test_library_loads_and_exports_header_symbols():
    L = hg.lib()
    syms = hg.declared_symbols()
    assert "hipgemm_fp8_gemm_bf16" in syms
    assert "hipgemm_fp8_gemm_4wave_256x256x128" in syms
    for s in syms:
        assert hasattr(L, s), s
    out = subprocess.run(["nm", "-D", "--defined-only", hg.lib_path()],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [s for s in syms if s not in exported]
    assert not missing, missing


def test_version_and_variants():
    assert hg.version() == 100
    assert hg.variant_name(0) == "auto"
    assert hg.variant_name(1).startswith("4wave")
    assert hg.variant_name(99) is None
    assert hg.variant_name(2).startswith("4wave")
    assert hg.variant_name(3).startswith("skinny")
    assert hg.variant_name(4).startswith("8wave")
    assert hg.variant_name(5).startswith("4wave_128x128")
    assert hg.variant_name(6).startswith("strip")
    assert hg.variant_name(7) is None
    assert hg.select_variant(8192, 8192, 8192) == 2
    assert hg.select_variant(4000, 5000, 3584) == 2
    # 128 x 128 tiles in one round over the (256, without a device) CUs
    assert hg.select_variant(2048, 2048, 2048) == 5
    assert hg.select_variant(512, 512, 512) == 5
    assert hg.select_variant(2048, 4096, 2048) == 5   # short K, 128 tiles
    assert hg.select_variant(2048, 4096, 4096) == 2   # 2 full rounds of 128x128
    assert hg.select_variant(1536, 4096, 4096) == 5   # 96 tiles, 1.5 rounds
    assert hg.select_variant(640, 8192, 8192) == 2    # the same with a side of 8192
    assert hg.select_variant(8192, 896, 4096) == 2
    assert hg.select_variant(640, 8192, 2048) == 5    # short K
    assert hg.select_variant(128, 8192, 8192) == 5   # 64 tiles x 4 K-slices
    assert hg.select_variant(80, 8192, 1024) == 6    # B_T of 8 MiB: strips
    assert hg.select_variant(96, 2048, 4096) == 6
    assert hg.select_variant(128, 4096, 4096) == 3   # half-filled K-split
    assert hg.select_variant(128, 8192, 2048) == 5   # ... of 2 slices only
    assert hg.select_variant(100, 1536, 8192) == 5   # 65-128 rows, N < 2048
    assert hg.select_variant(120, 2560, 4096) == 3
    assert hg.select_variant(65, 2048, 8192) == 3
    # up to 64 rows: column strips, but 128 x 128 tiles for very wide N with
    # short K, and above 40 rows for long K
    assert hg.select_variant(64, 8192, 8192) == 6
    assert hg.select_variant(64, 4096, 4096) == 6
    assert hg.select_variant(64, 2048, 2048) == 6
    assert hg.select_variant(48, 1024, 1024) == 5    # K <= 1024, 32 strips
    assert hg.select_variant(48, 8192, 1024) == 6    # ... 256 strips
    assert hg.select_variant(40, 2048, 1024) == 5    # ... 64 strips: a quarter
    assert hg.select_variant(40, 3072, 1024) == 6    # ... 96 strips
    assert hg.select_variant(32, 1024, 1024) == 6
    assert hg.select_variant(16, 8192, 8192) == 6
    assert hg.select_variant(16, 28672, 1024) == 6   # 16 rows: strips throughout
    assert hg.select_variant(24, 28672, 2048) == 5
    assert hg.select_variant(24, 28672, 4096) == 5   # from 17 rows, any K
    assert hg.select_variant(40, 28672, 4096) == 5
    assert hg.select_variant(40, 28672, 8192) == 5
    assert hg.select_variant(28, 20480, 1536) == 5   # N > 64 x CUs
    assert hg.select_variant(36, 20480, 6144) == 5
    assert hg.select_variant(36, 20480, 12288) == 5
    assert hg.select_variant(36, 16384, 2048) == 6
    assert hg.select_variant(64, 8192, 14336) == 5   # 41-64 rows, long K
    assert hg.select_variant(48, 8192, 14336) == 6   # 33-48 rows: strip
    assert hg.select_variant(40, 8192, 14336) == 6   # 40 rows: strip
    assert hg.select_variant(48, 4096, 8192) == 6    # K = 8192: strip
    assert hg.select_variant(48, 3072, 10240) == 6
    assert hg.select_variant(52, 3072, 10240) == 5
    assert hg.select_variant(64, 2048, 14336) == 6   # N < 3072
    assert hg.select_variant(129, 8192, 8192) == 5   # 2 x 64 tiles of 128


def test_tile128_k_split_workspace():
    """The 128 x 128 schedule splits K when its tiles fill at most a quarter
    of the (256) CUs and K has 16+ steps: 256 x 4096 x 14336 is 2 x 32 tiles,
    4 slices of 28 steps, one 64 KiB partial per (tile, slice), after the
    counter region every workspace starts with (HIPGEMM_WS_COUNTER_BYTES).
    At most half of them and 64+ steps: 2 slices."""
    ctr = 16384
    assert hg.workspace_size(256, 4096, 14336, 5) == ctr + 64 * 4 * 65536
    assert hg.workspace_size(256, 4096, 14336, 0) == ctr + 64 * 4 * 65536  # AUTO
    assert hg.workspace_size(256, 8192, 8192, 5) == ctr + 128 * 2 * 65536
    assert hg.workspace_size(256, 8192, 4096, 5) == 0    # 128 tiles, 32 steps
    assert hg.workspace_size(384, 4096, 8192, 5) == ctr + 96 * 2 * 65536
    assert hg.workspace_size(512, 8192, 8192, 5) == 0    # 256 tiles
    assert hg.workspace_size(256, 4096, 1920, 5) == 0    # 15 steps: no split
    # 300 x 1000 x 4112: 3 x 8 tiles, 33 steps -> 4 slices of 10 steps
    assert hg.workspace_size(300, 1000, 4112, 5) == ctr + 24 * 4 * 65536


def test_workspace_counter_region():
    """Every schedule's workspace starts with the same counter region; the
    skinny schedule's partial tiles follow it (128 x 8192 x 8192: 64 column
    tiles of 128 x 4 K-slices, 64 KiB each)."""
    ctr = 16384
    text = open(hg._HEADER).read()
    assert f"#define HIPGEMM_WS_COUNTER_BYTES {ctr}" in text
    assert hg.workspace_size(128, 8192, 8192, 3) == ctr + 64 * 4 * 65536
    # 16 rows: 32 tiles of 256 columns x 8 slices, 16 x 256 fp32 each
    assert hg.workspace_size(16, 8192, 8192, 3) == ctr + 32 * 8 * 16384


def test_split_columns_plan():
    """AUTO's column split (256 CUs without a device): 4000 x 5000 has 16 x
    20 tiles of 256 = 1.25 rounds; 16 tile columns fill one round, the other
    904 columns are 32 x 8 = 256 tiles of 128, one round."""
    assert hg.split_columns(4000, 5000, 3584) == 4096
    for shape in [(8192, 8192, 8192), (4096, 4096, 4096), (2048, 2048, 2048),
                  (8192, 28672, 8192), (128, 8192, 8192), (6144, 6144, 4096),
                  (4000, 5000, 0)]:
        assert hg.split_columns(*shape) == 0, shape


@pytest.mark.parametrize("args", [
    dict(A=0),                         # null A
    dict(B=0),                         # null B_T
    dict(C=0),                         # null C
    dict(M=-1), dict(N=-5), dict(K=-16),
    dict(K=40, lda=48, ldb=48),        # K % 16 != 0
    dict(lda=48),                      # lda < K
    dict(ldb=48),                      # ldb < K
    dict(lda=72),                      # lda % 16 != 0
    dict(ldc=63),                      # ldc < N
    dict(A=FAKE + 8),                  # A not 16-byte aligned
    dict(B=FAKE + 4),                  # B_T not 16-byte aligned
    dict(C=FAKE + 1),                  # C not 2-byte aligned
    dict(lda=(1 << 23) + 16),          # lda too large for 32-bit offsets
    dict(ldc=(1 << 22) + 4),           # ldc too large for 32-bit offsets
    dict(variant=7), dict(variant=-1),
])
def test_argument_validation(args):
    p = dict(A=FAKE, B=FAKE, C=FAKE, M=64, N=64, K=64, lda=64, ldb=64, ldc=64,
             variant=0)
    p.update(args)
    code = hg.gemm_raw(p["A"], p["B"], p["C"], p["M"], p["N"], p["K"],
                       p["lda"], p["ldb"], p["ldc"], 0, 0, p["variant"], 0)
    assert code == INVALID


def test_empty_problem_is_a_noop():
    assert hg.gemm_raw(0, 0, 0, 0, 64, 64, 64, 64, 64) == 0
    assert hg.gemm_raw(0, 0, 0, 64, 0, 64, 64, 64, 64) == 0


def test_k_zero_needs_only_c():
    # K == 0 does not read A / B_T, so they may be NULL; C is still checked.
    assert hg.gemm_raw(0, 0, 0, 64, 64, 0, 0, 0, 64) == INVALID
    assert hg.gemm_raw(0, 0, FAKE + 1, 64, 64, 0, 0, 0, 64) == INVALID
    assert hg.gemm_raw(0, 0, FAKE, 64, 64, 0, 0, 0, 63) == INVALID


def test_workspace_size_and_validation():
    """The split-K schedule (M <= 128) needs a workspace when it splits K;
    the workspace entry point rejects a missing, misaligned or short one
    before launching anything."""
    skinny = hg.VARIANTS["skinny"]
    strip = hg.VARIANTS["strip"]
    assert hg.select_variant(100, 4096, 4096) == skinny
    assert hg.select_variant(129, 8192, 8192) != skinny
    need = hg.workspace_size(100, 4096, 4096, 0)
    assert need > 0 and need % 256 == 0
    assert hg.workspace_size(100, 4096, 4096, skinny) == need
    # The strip schedule needs none when N / 32 fills the (256) CUs, and
    # counters plus 2 slices x 128 strips x 16 x 32 fp32 at N = 4096.
    assert hg.workspace_size(16, 8192, 8192, 0) == 0
    assert hg.workspace_size(16, 4096, 8192, strip) == 16384 + 2 * 128 * 2048
    assert hg.workspace_size(512, 8192, 8192, 0) == 0   # 4-wave: none
    assert hg.workspace_size(16, 300, 64, 0) == 0       # one K-step: no split
    assert hg.workspace_size(0, 8192, 8192, 0) == 0
    args = (FAKE, FAKE, FAKE, 100, 4096, 4096, 4096, 4096, 4096, 0, 0)
    assert hg.gemm_raw_ws(*args, 0, 0, need) == INVALID          # no workspace
    assert hg.gemm_raw_ws(*args, 0, FAKE, need - 256) == INVALID  # too small
    assert hg.gemm_raw_ws(*args, 0, FAKE + 64, need) == INVALID   # misaligned
    assert hg.gemm_raw_ws(*args[:3], 129, *args[4:], skinny, FAKE,
                          need) == INVALID                       # M > 128
    assert hg.gemm_raw_ws(0, 0, 0, 0, 8192, 8192, 8192, 8192, 8192, 0, 0, 0,
                          0, 0) == 0                             # empty: no-op


def test_rowcol_entry_validation():
    """The per-row / per-column entry point: the common argument checks, plus
    4-byte aligned vectors and no 32x32x64 schedule; NULL vectors are
    accepted (all ones) and empty problems are no-ops."""
    base = dict(A=FAKE, B=FAKE, C=FAKE, M=300, N=300, K=64, lda=64, ldb=64,
                ldc=300, rows=FAKE, cols=FAKE, variant=0)

    def call(**kw):
        p = dict(base)
        p.update(kw)
        return hg.gemm_raw_rowcol(p["A"], p["B"], p["C"], p["M"], p["N"],
                                  p["K"], p["lda"], p["ldb"], p["ldc"],
                                  p["rows"], p["cols"], p["variant"], 0, 0, 0)

    for bad in (dict(rows=FAKE + 2), dict(cols=FAKE + 1),
                dict(variant=hg.VARIANTS["4wave"]), dict(variant=7),
                dict(variant=hg.VARIANTS["strip"]),  # M = 300 > 128
                dict(K=40, lda=48, ldb=48), dict(ldc=299), dict(A=0),
                dict(variant=hg.VARIANTS["skinny"])):  # M = 300 > 128
        assert call(**bad) == INVALID, bad
    assert call(M=0) == 0 and call(N=0, rows=FAKE + 2) == 0
    args = (FAKE, FAKE, FAKE, 16, 8192, 8192, 8192, 8192, 8192, 0, 0,
            hg.VARIANTS["skinny"])
    need = hg.workspace_size(16, 8192, 8192, hg.VARIANTS["skinny"])
    assert hg.gemm_raw_rowcol(*args, 0, need) == INVALID          # missing
    assert hg.gemm_raw_rowcol(*args, FAKE, need - 256) == INVALID  # short
    assert hg.gemm_raw_rowcol(*args, FAKE + 64, need) == INVALID   # misaligned


def test_gemm_desc_entry_validation():
    """hipgemm_gemm: the descriptor's size must match (a size-0 problem with
    the right size is a no-op, so the ctypes layout is the C one); codes,
    vector alignment and the 32x32x64 schedule's limits are checked before
    any HIP call."""
    base = dict(A=FAKE, B_T=FAKE, C=FAKE, M=300, N=300, K=64, lda=64, ldb=64,
                ldc=300)
    assert hg.gemm_desc_raw(hg.GemmDesc(**dict(base, M=0))) == 0
    bad_size = hg.GemmDesc(**base)
    bad_size.size -= 8
    assert hg.gemm_desc_raw(bad_size) == INVALID
    assert hg.lib().hipgemm_gemm(None, None) == INVALID
    for bad in (dict(a_format=2), dict(b_format=-1), dict(out_dtype=4),
                dict(out_dtype=-1), dict(activation=4), dict(scale_rows=FAKE + 2),
                # fp32 / e4m3 output: element alignment, no 8-wave schedule,
                # the output scale only with e4m3 output, 4-byte aligned
                dict(out_dtype=2, C=FAKE + 2), dict(out_dtype=2, variant=4),
                dict(out_dtype=3, variant=4), dict(scale_out=FAKE),
                dict(out_dtype=2, scale_out=FAKE),
                dict(out_dtype=3, scale_out=FAKE + 2),
                # ldc * element size <= 2^23 bytes
                dict(out_dtype=2, ldc=(1 << 21) + 1),
                dict(scale_cols=FAKE + 1), dict(bias=FAKE + 3),
                dict(variant=1, a_format=1), dict(variant=1, bias=FAKE),
                dict(variant=1, out_dtype=1), dict(variant=1, activation=1),
                dict(variant=3),  # M = 300 > 128
                dict(K=40, lda=48, ldb=48), dict(variant=9)):
        assert hg.gemm_desc_raw(hg.GemmDesc(**dict(base, **bad))) == INVALID, bad
    # e4m3 output: any byte address; the empty problem is a no-op
    assert hg.gemm_desc_raw(hg.GemmDesc(**dict(base, M=0, out_dtype=3,
                                               C=FAKE + 1))) == 0


def test_fp4_entry_validation():
    """fp4 operands: both fp4, K (elements) a multiple of 32, lda / ldb in
    bytes >= K / 2; AUTO, the 128 x 128 schedule or the 4-wave 16x16x128
    one (MX scales on either, with the per-tensor epilogue).  The
    descriptor's workspace query plans the
    128 x 128 schedule on K / 2 bytes, and nothing where AUTO takes the
    4-wave schedule."""
    base = dict(A=FAKE, B_T=FAKE, C=FAKE, M=300, N=300, K=256, lda=128,
                ldb=128, ldc=300, a_format=4, b_format=4)
    assert hg.gemm_desc_raw(hg.GemmDesc(**dict(base, M=0))) == 0
    for bad in (dict(b_format=0), dict(a_format=1), dict(K=240), dict(lda=112),
                dict(variant=1), dict(variant=3), dict(variant=4),
                dict(mx_scale_a=FAKE, mx_scale_b=FAKE, variant=2, bias=FAKE),
                dict(mx_scale_a=FAKE, mx_scale_b=FAKE, bias=FAKE)):
        assert hg.gemm_desc_raw(hg.GemmDesc(**dict(base, **bad))) == INVALID, bad
    L = hg.lib()
    # 256 x 4096 x 28672 elements = 14336 bytes per row: 2 x 32 tiles of 128,
    # 112 steps -> 4 slices of 28 steps (as for 8-bit K = 14336)
    d = hg.GemmDesc(**dict(base, M=256, N=4096, K=28672, lda=14336, ldb=14336,
                           ldc=4096))
    assert L.hipgemm_gemm_workspace_size(ctypes.byref(d)) == \
        hg.workspace_size(256, 4096, 14336, 5) == 16384 + 64 * 4 * 65536
    d8 = hg.GemmDesc(**dict(base, a_format=0, b_format=0, M=256, N=4096,
                            K=14336, lda=14336, ldb=14336, ldc=4096))
    assert L.hipgemm_gemm_workspace_size(ctypes.byref(d8)) == 16384 + 64 * 4 * 65536
    # 8192^3 elements: AUTO takes the 4-wave schedule, which needs none
    big = hg.GemmDesc(**dict(base, M=8192, N=8192, K=8192, lda=4096, ldb=4096,
                             ldc=8192))
    assert L.hipgemm_gemm_workspace_size(ctypes.byref(big)) == 0


def test_fp6_entry_validation():
    """fp6 operands: both fp6 (either variant each), K (elements) a multiple
    of 64, lda / ldb in bytes >= 3K / 4, AUTO, the 128 x 128 schedule or
    the 4-wave 16x16x128 one, no MX scales; the
    descriptor's workspace query plans the 128 x 128 schedule on 96-byte
    steps of 3K / 4 bytes where it runs, and the 4-wave one needs none."""
    base = dict(A=FAKE, B_T=FAKE, C=FAKE, M=300, N=300, K=256, lda=192,
                ldb=192, ldc=300, a_format=2, b_format=3)
    assert hg.gemm_desc_raw(hg.GemmDesc(**dict(base, M=0))) == 0
    for bad in (dict(b_format=0), dict(a_format=1), dict(a_format=4),
                dict(K=224), dict(lda=176), dict(variant=1), dict(variant=3),
                dict(variant=4), dict(variant=6),
                dict(mx_scale_a=FAKE, mx_scale_b=FAKE)):
        assert hg.gemm_desc_raw(hg.GemmDesc(**dict(base, **bad))) == INVALID, bad
    L = hg.lib()
    # 256 x 2048 x 3072 elements = 2304 bytes per row: 2 x 16 tiles of 128,
    # 24 steps of 96 bytes -> 3 slices of 8 steps
    d = hg.GemmDesc(**dict(base, M=256, N=2048, K=3072, lda=2304, ldb=2304,
                           ldc=2048))
    assert L.hipgemm_gemm_workspace_size(ctypes.byref(d)) == 16384 + 32 * 3 * 65536
    # AUTO takes the 4-wave schedule (no workspace) where it does for 8-bit
    # operands of the byte shape, with either epilogue
    big = dict(base, M=4096, N=4096, K=4096, lda=3072, ldb=3072, ldc=4096)
    assert hg.select_variant(4096, 4096, 3072) == 2
    assert L.hipgemm_gemm_workspace_size(ctypes.byref(hg.GemmDesc(**big))) == 0
    assert L.hipgemm_gemm_workspace_size(
        ctypes.byref(hg.GemmDesc(**dict(big, variant=2)))) == 0
    assert L.hipgemm_gemm_workspace_size(
        ctypes.byref(hg.GemmDesc(**dict(big, out_dtype=2, bias=FAKE)))) == 0


def test_mx_entry_validation():
    """MX block scales: packed size, packing arguments, and the descriptor
    rules (both scales, K % 32, 16-byte alignment, no extended epilogue,
    the 4-wave 16x16x128 schedule or AUTO) -- all before any HIP call."""
    assert hg.mx_scales_bytes(0, 256) == 0 and hg.mx_scales_bytes(100, 0) == 0
    # ceil(rows/128) groups x ceil(ceil(K/128)/2) step pairs x 1 KiB
    assert hg.mx_scales_bytes(128, 256) == 1024
    assert hg.mx_scales_bytes(129, 384) == 2 * 2 * 1024
    assert hg.mx_scales_bytes(8192, 8192) == 64 * 32 * 1024 == 8192 * 8192 // 32
    L = hg.lib()
    assert L.hipgemm_mx_pack_scales(FAKE, 64, 48, 2, FAKE, None) == INVALID   # K % 32
    assert L.hipgemm_mx_pack_scales(FAKE, 64, 64, 1, FAKE, None) == INVALID   # ld < K/32
    assert L.hipgemm_mx_pack_scales(None, 64, 64, 2, FAKE, None) == INVALID
    assert L.hipgemm_mx_pack_scales(None, 0, 64, 2, None, None) == 0          # empty
    base = dict(A=FAKE, B_T=FAKE, C=FAKE, M=300, N=300, K=64, lda=64, ldb=64,
                ldc=300, mx_scale_a=FAKE, mx_scale_b=FAKE)
    assert hg.gemm_desc_raw(hg.GemmDesc(**dict(base, M=0))) == 0
    for bad in (dict(mx_scale_b=0), dict(mx_scale_a=0, mx_scale_b=FAKE),
                dict(K=48, lda=48, ldb=48), dict(mx_scale_a=FAKE + 8),
                dict(bias=FAKE), dict(scale_rows=FAKE), dict(out_dtype=1),
                dict(activation=1), dict(variant=1), dict(variant=3),
                dict(variant=4)):
        assert hg.gemm_desc_raw(hg.GemmDesc(**dict(base, **bad))) == INVALID, bad


def test_dropin_entry_validates_too():
    L = hg.lib()
    assert L.hipgemm_fp8_gemm_4wave_256x256x128(None, None, None, 64, 64, 64,
                                                None) == INVALID
    assert L.hipgemm_fp8_gemm_4wave_256x256x128(FAKE, FAKE, FAKE, 64, 64, 40,
                                                None) == INVALID


def test_missing_library_fails_loudly(tmp_path):
    code = (
        "import hipgemm_amd as h\n"
        "h._LIB_PATH = '/nonexistent/libhipgemm.so'\n"
        "try:\n"
        "    h.lib()\n"
        "except h.HipGemmError as e:\n"
        "    print('raised', e)\n"
        "else:\n"
        "    raise SystemExit('no error')\n")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", code], cwd=root,
                       capture_output=True, text=True)
    assert r.returncode == 0 and "raised" in r.stdout, r.stderr


def test_product_does_not_import_oracle():
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    pkg = os.path.join(root, "hipgemm_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".cpp", ".hpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in text.replace("oracle/", ""), f
    for dirpath, _, files in os.walk(os.path.join(root, "include")):
        for f in files:
            assert "oracle" not in open(os.path.join(dirpath, f)).read(), f


def test_mfma_ceiling_probe_library():
    """bench.py's MFMA ceiling probe is its own library (nothing of it is in
    libhipgemm.so): it loads, exports its two entry points, reads 2 MiB of
    operands (64 sets x 16 fragments x 64 lanes x 32 bytes) and rejects bad
    arguments before launching."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    path = os.path.join(root, "hipgemm_amd", "libhipgemm_probe.so")
    L = ctypes.CDLL(path)
    L.hipgemm_probe_ops_bytes.restype = ctypes.c_size_t
    assert L.hipgemm_probe_ops_bytes() == 64 * 16 * 64 * 32
    f = L.hipgemm_probe_mfma_ceiling
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                  ctypes.c_void_p]
    f.restype = ctypes.c_int
    assert f(None, None, 256, 256, None) == INVALID
    assert f(FAKE, FAKE, 0, 256, None) == INVALID
    assert f(FAKE, FAKE, 256, 0, None) == INVALID
    assert not hasattr(hg.lib(), "hipgemm_probe_mfma_ceiling")


def test_bench_gpu_monitor_window():
    """bench.py's clock/power monitor: window() averages the samples between
    two host times (mean clock, its range, mean power) and gives None for an
    empty window; without a GPU the monitor starts, stops and reports
    nothing rather than failing the bench."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    sys.path.insert(0, root)
    import bench
    m = bench.GpuMonitor.__new__(bench.GpuMonitor)
    m.cap_w = 1400.0
    m.samples = [(1.0, 2000.0, 1000.0), (2.0, 1800.0, 1400.0),
                 (3.0, 1700.0, None), (9.0, 100.0, 10.0)]
    w = m.window(1.5, 3.5)
    assert w == {"gfxclk_mhz": 1750.0, "gfxclk_mhz_range": [1700.0, 1800.0],
                 "socket_power_w": 1400.0, "power_cap_w": 1400.0,
                 "samples": 2}
    assert m.window(4.0, 8.0) is None
    import torch
    if not torch.cuda.is_available():
        g = bench.GpuMonitor(0).start()
        g.stop()
        assert not g.ok and g.window(0.0, 1e18) is None


def test_sweep_shape_parser():
    from hipgemm_amd import sweep
    assert sweep.parse_shapes("64x4096x4096,1X2x3") == [(64, 4096, 4096), (1, 2, 3)]
    with pytest.raises(ValueError):
        sweep.parse_shapes("0x1x1")
    with pytest.raises(ValueError):
        sweep.parse_shapes("64x4096")
    assert sweep.parse_grid("16,32:4096:1024,2048") == [
        (16, 4096, 1024), (16, 4096, 2048), (32, 4096, 1024), (32, 4096, 2048)]
    with pytest.raises(ValueError):
        sweep.parse_grid("16:4096")


def test_auto_picks_fit_their_shape_and_the_noalloc_scratch():
    """Over a grid of shapes: AUTO picks one of the schedules it documents
    (never the 32x32x64 or 8-wave ones), the skinny-M schedules only up to
    128 rows, and the workspace its pick needs fits the no-allocation
    entry point's static scratch (HIPGEMM_NOALLOC_SCRATCH_BYTES), so that
    entry point takes every shape AUTO does.  (On the CPU the library
    assumes 256 CUs.)"""
    scratch = (16 << 10) + (32 << 20)
    V = hg.VARIANTS
    rows = [1, 8, 16, 17, 24, 32, 33, 40, 41, 48, 56, 64, 65, 72, 96, 100, 128,
            129, 200, 256, 384, 512, 640, 1024, 1536, 2048, 4000, 8192]
    cols = [16, 512, 1000, 1024, 1536, 2048, 3072, 4096, 5000, 6144, 8192,
            12288, 16384, 17408, 20480, 28672, 32768]
    ks = [16, 128, 1024, 2048, 3072, 4096, 6144, 8192, 12288, 14336, 28672]
    for M in rows:
        for N in cols:
            for K in ks:
                v = hg.select_variant(M, N, K)
                assert v in (V["4wave_mfma16"], V["tile128"], V["skinny"], V["strip"]), (M, N, K, v)
                if v in (V["skinny"], V["strip"]):
                    assert M <= 128, (M, N, K, v)
                ws = hg.workspace_size(M, N, K, 0)
                assert ws == hg.workspace_size(M, N, K, v), (M, N, K)
                assert ws <= scratch, (M, N, K, v, ws)
