"""The static launch-shape table: key format, M buckets, lookup, and the
committed gfx950 table's entries being valid launch shapes (CPU)."""

from __future__ import annotations

import json

import torch

from breeze_amd import tuning


def test_buckets_and_keys():
    assert [tuning.m_bucket(m) for m in (1, 2, 3, 4, 5, 8, 9, 16, 17, 100)] == [1, 2, 4, 4, 8, 8, 16, 16, 32, 32]
    assert tuning.table_key("gfx950", 4096, 2048, 0, 1, True, 2) == "gfx950|4096|2048|0|1|1|2"


def test_lookup_reads_the_table(monkeypatch, tmp_path):
    path = tmp_path / "t.json"
    path.write_text(json.dumps({"gfx950|64|256|0|0|1|2": [2, 8, 0, 1]}))
    monkeypatch.setenv("BZ_TUNE_TABLE", str(path))
    monkeypatch.setattr(tuning, "_TABLES", {})
    monkeypatch.setattr(tuning, "arch_of", lambda dev: "gfx950")
    dev = torch.device("cpu")
    assert tuning.lookup(dev, 64, 256, 0, 0, True, 2) == (2, 8, 0, 1)
    assert tuning.lookup(dev, 64, 256, 0, 0, True, 1) is None
    assert tuning.lookup(dev, 64, 256, 0, 0, False, 2) is None


def test_committed_table_entries_are_valid_shapes():
    table = json.loads((tuning.PKG_DIR / "tune_gfx950.json").read_text())
    assert table
    for key, cfg in table.items():
        arch, N, K, wfmt, epi, norm, mb = key.split("|")
        assert arch == "gfx950" and int(mb) in (1, 2, 4, 8, 16, 32)
        assert len(cfg) in (4, 5)
        depth, waves, tiles, path = cfg[:4]
        # 0 = the built-in choice for that field
        if path == 6:  # the panel kernel: unpaired tiled weights, no prologue or epilogue but the
            # residual; waves <= 16 (<= 8 with several blocks), 1-5 row blocks per workgroup
            assert int(wfmt) in (4, 6) and not int(norm) and int(epi) in (0, 2) and depth == 0
            assert 1 <= tiles <= 5 and 0 <= waves <= (16 if tiles == 1 else 8) and len(cfg) == 4
            continue
        if path == 5:  # the streaming kernels of the tiled formats: the wave count, and the row
            # blocks per workgroup (0: the one-block kernel, 1-8: the several-block kernel)
            assert int(wfmt) in (4, 5, 6, 7) and 1 <= waves <= 16 and depth == 0 and 0 <= tiles <= 8
            assert len(cfg) == 4
            continue
        # row-major formats; path 4 also reads the unpaired tiled ones in place
        assert int(wfmt) in (0, 1, 2, 3) or (path == 4 and int(wfmt) in (4, 6))
        assert depth in (0, 2, 4, 8, 16) and 0 <= waves <= 8 and tiles >= 0 and path in (1, 2, 3, 4)
        if path == 3:
            assert int(wfmt) in (0, 1)  # int8 matrix-core path is for int4 weights only
        if path == 4:  # several-row tile kernel: no prologue or SiLU gate, 4 or 8 waves, 1 or 2 tiles
            assert norm == "0" and epi != "1" and waves in (0, 4, 8) and tiles in (0, 1, 2) and depth <= 8
            assert len(cfg) == 5 and cfg[4] >= 0
        else:
            assert len(cfg) == 4 or cfg[4] == 0
