"""The C ABI: librfill.so loads without a GPU and exports every entry point include/rfill.h declares,
and the Python binding declares exactly those (no compute calls here)."""
import ctypes

import pytest
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def declared():
    text = (ROOT / "include" / "rfill.h").read_text()
    return sorted(set(re.findall(r"^(?:int|const char\*)\s+(rf_\w+)\s*\(", text, re.M)))


def test_header_declares_the_entry_points():
    names = declared()
    assert "rf_map_apply" in names and "rf_norm_kv_write" in names and "rf_last_error" in names


def test_library_exports_every_declared_symbol():
    from rfill import _lib
    assert _lib.LIB_PATH.exists(), "librfill.so not built: run __graft_entry__.build()"
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing
    assert lib.rf_version() >= 1


def test_binding_covers_the_header():
    from rfill import _lib
    compute = [n for n in declared() if n not in ("rf_last_error", "rf_version")]
    assert sorted(_lib.SIGNATURES) == compute


def test_status_codes_match_the_header():
    from rfill import _lib
    text = (ROOT / "include" / "rfill.h").read_text()
    for name in ("RF_OK", "RF_EINVAL_SHAPE", "RF_EINVAL_ARG", "RF_EUNSUPPORTED", "RF_EHIP"):
        value = int(re.search(rf"#define {name} \(?(-?\d+)\)?", text).group(1))
        assert getattr(_lib, name) == value
    assert _lib.SSQ_COLS == int(re.search(r"#define RF_SSQ_COLS (\d+)", text).group(1))


def test_gemm_workspace_sizes():
    """Host-only size rule of the GEMM entry points' split-K workspace: splits x M x N fp32. Products of at
    most 512 rows (the few-rows kernel: row blocks of <= 160 rows x 256 columns)
    always take it, splits = max(1, min(256 / blocks, K / 512, 16)); otherwise when the 256 x 256 tiles are
    too few for the GPU (splits = min(256 / tiles, K / 512, 16)), or the last wave's tile rows, else none."""
    from rfill import ops
    assert ops.gemm_workspace_bytes(28672, 4096, 4096) == 0          # the fill: 1792 tiles, unsplit
    assert ops.gemm_workspace_bytes(287, 4096, 4096) == 8 * 287 * 4096 * 4       # 2 x 16 blocks: 8 splits
    assert ops.gemm_workspace_bytes(287, 24576, 4096) == 287 * 24576 * 4         # 2 x 96 blocks: one split
    assert ops.gemm_workspace_bytes(123, 4096, 4096) == 8 * 123 * 4096 * 4       # 1 x 16 blocks: K / 512 = 8
    assert ops.gemm_workspace_bytes(513, 4096, 4096) == 5 * 513 * 4096 * 4       # 3 x 16 tiles of 256 x 256
    assert ops.gemm_workspace_bytes(4096, 2048, 4096) == 2 * 4096 * 2048 * 4     # the tail's K / V: 128 tiles
    # the fill's K / V: 896 tiles = 3 waves + 16 tile rows (128 tiles): those rows split 2 ways
    assert ops.gemm_workspace_bytes(28672, 2048, 4096) == 2 * 4096 * 2048 * 4
    assert ops.gemm_workspace_bytes(28672, 1024, 2048) == 0          # 48 of 64 tile rows in the last wave
    assert ops.gemm_workspace_bytes(40, 512, 2048) == 4 * 40 * 512 * 4           # K / 512 = 4 caps the splits
    assert ops.gemm_workspace_bytes(287, 4096, 256) == 287 * 4096 * 4            # few rows: one split
    assert ops.gemm_workspace_bytes(600, 4096, 256) == 0             # too little K to split
    assert ops.gemm_workspace_bytes(0, 4096, 4096) == 0
    with pytest.raises(ValueError):
        ops.gemm_workspace_bytes(10, 100, 4096)                     # N not a multiple of 256


def test_rows_workspace_sizes():
    """Host-only size rule of the scattered rows' K / V products (rf_norm_kv_rows, rf_norm_qkv_rows): they
    run 512 rows at a time, each chunk planned alone, so the workspace is the largest chunk's. At Qwen3-8B
    widths ([wq; wkv]: N 6144, K 4096) a full chunk takes 4 row blocks x 24 column blocks, K split 2 ways;
    655 rows leave a last chunk of 143 rows in one row block, split min(256 / 24, K / 512) = 8 ways, which
    needs more than the full chunk."""
    from rfill import ops
    full = 2 * 512 * 6144 * 4
    assert ops.rows_workspace_bytes(512, 6144, 4096) == full
    assert ops.rows_workspace_bytes(655, 6144, 4096) == 8 * 143 * 6144 * 4 > full
    assert ops.rows_workspace_bytes(1024, 6144, 4096) == full
    assert ops.rows_workspace_bytes(287, 2048, 4096) == 8 * 287 * 2048 * 4      # one chunk: as the GEMM's
    assert ops.rows_workspace_bytes(0, 2048, 4096) == 0
    # every chunk of every row count fits, at the widths the exact rows use
    for n, k in ((6144, 4096), (2048, 4096), (4608, 2048), (1024, 1024)):
        for rows in range(1, 2100, 7):
            need = ops.rows_workspace_bytes(rows, n, k)
            chunks = [512] * (rows // 512) + ([rows % 512] if rows % 512 else [])
            assert need == max(ops.gemm_workspace_bytes(m, n, k) for m in chunks), (n, k, rows)
    with pytest.raises(ValueError):
        ops.rows_workspace_bytes(10, 100, 4096)


def test_gram_workspace_sizes():
    """Host-only size rule of rf_gram_accumulate's run-split schedule: when the 256 x 256 tiles are more than
    256 but fewer than 512 and K holds two or more runs, the tiles past the first 256 are cut into their runs
    (at most 512 of them), each stored as a 256 x 256 fp32 plane; otherwise no workspace."""
    from rfill import ridge
    plane = 256 * 256 * 4
    assert ridge.gram_workspace_bytes(4096, 4096, 65536, 8192) == 0          # 256 tiles: one round
    assert ridge.gram_workspace_bytes(4104, 4352, 65536, 8192) == 33 * 8 * plane   # centred X and Y: 289 tiles
    assert ridge.gram_workspace_bytes(4104, 4096, 65536, 8192) == 16 * 8 * plane   # centred X only: 272 tiles
    assert ridge.gram_workspace_bytes(4104, 4352, 12288, 8192) == 33 * 2 * plane   # a short last run counts
    assert ridge.gram_workspace_bytes(4104, 4352, 65536, 0) == 0             # one run: nothing to split
    assert ridge.gram_workspace_bytes(4104, 4352, 65536, 4096) == 0          # 33 x 16 = 528 runs > 512: whole
    assert ridge.gram_workspace_bytes(5120, 5120, 65536, 8192) == 0          # 400 tiles, 1152 runs: whole
    assert ridge.gram_workspace_bytes(8192, 8192, 65536, 8192) == 0          # 1024 tiles: whole rounds
    assert ridge.gram_workspace_bytes(0, 4096, 65536, 8192) == 0
    with pytest.raises(ValueError):
        ridge.gram_workspace_bytes(4096, 100, 65536, 8192)                  # N not a multiple of 256


def test_gram_upper_workspace_sizes():
    """Host-only size rule of rf_gram_accumulate_upper: the block-upper tiles (tile column >= tile row), when
    at most one round of them and K holds two or more runs, all split into their runs; past one round, the
    rule of rf_gram_accumulate over that tile count."""
    from rfill import ridge
    plane = 256 * 256 * 4
    assert ridge.gram_upper_workspace_bytes(4096, 4096, 65536, 8192) == 136 * 8 * plane   # 16 x 16 tiles
    assert ridge.gram_upper_workspace_bytes(4104, 4352, 65536, 8192) == 153 * 8 * plane   # centred X: 17 x 17
    assert ridge.gram_upper_workspace_bytes(5120, 5120, 65536, 8192) == 210 * 8 * plane   # 20 x 20
    assert ridge.gram_upper_workspace_bytes(4096, 4096, 12288, 8192) == 136 * 2 * plane   # a short last run
    assert ridge.gram_upper_workspace_bytes(4096, 4096, 65536, 0) == 0      # one run: nothing to split
    assert ridge.gram_upper_workspace_bytes(8192, 8192, 65536, 8192) == 0   # 528 tiles: whole rounds
    assert ridge.gram_upper_workspace_bytes(0, 4096, 65536, 8192) == 0
    with pytest.raises(ValueError):
        ridge.gram_upper_workspace_bytes(4352, 4096, 65536, 8192)           # M past N
