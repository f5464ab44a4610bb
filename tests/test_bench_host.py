"""CPU: the bench's stamp of the HBM-traffic figure (bench.kernel_source_sha,
bench.read_traffic).

The traffic figure comes from counter runs recorded in profiles/ with the
hash of the kernel sources they were taken on; bench.py reports it only
while the sources it runs hash the same.  The hash covers the sources'
code: a comment or whitespace edit keeps it, a code edit changes it, and a
stale summary is reported as absent, with the reason.
"""

from __future__ import annotations

import shutil
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(REPO))

import bench  # noqa: E402


def _copy_sources(dst: Path) -> Path:
    (dst / "dsa-multi-layer-indexer_amd").mkdir(parents=True)
    shutil.copytree(REPO / "dsa-multi-layer-indexer_amd" / "csrc", dst / "dsa-multi-layer-indexer_amd" / "csrc")
    (dst / "include").mkdir()
    shutil.copy(REPO / "include" / "dsa_mli.h", dst / "include" / "dsa_mli.h")
    return dst


def test_hash_ignores_comments_and_whitespace(tmp_path):
    root = _copy_sources(tmp_path / "a")
    base = bench.kernel_source_sha(root)
    assert base == bench.kernel_source_sha()
    f = root / "dsa-multi-layer-indexer_amd" / "csrc" / "scan_flat.hip"
    text = f.read_text()
    f.write_text("// a new comment line\n" + text.replace("\n\n", "\n  \n\n", 3) + "\n/* trailing\n block */\n")
    assert bench.kernel_source_sha(root) == base


@pytest.mark.parametrize("edit", ["constant", "header"])
def test_hash_follows_code(tmp_path, edit):
    root = _copy_sources(tmp_path / "b")
    base = bench.kernel_source_sha(root)
    if edit == "constant":
        f = root / "dsa-multi-layer-indexer_amd" / "csrc" / "scan_flat.hip"
        text = f.read_text()
        assert "kFlatBufBatches = 256" in text
        f.write_text(text.replace("kFlatBufBatches = 256", "kFlatBufBatches = 128", 1))
    else:
        f = root / "include" / "dsa_mli.h"
        f.write_text(f.read_text() + "\nint dsa_extra_symbol(void);\n")
    assert bench.kernel_source_sha(root) != base


def test_stale_traffic_summary_is_not_reported(tmp_path, monkeypatch):
    current = bench.TRAFFIC_FILE.read_text()
    stale = tmp_path / "traffic.md"
    lines = [l if not l.startswith("kernel_source_sha:") else "kernel_source_sha: 0000000000000000"
             for l in current.splitlines()]
    stale.write_text("\n".join(lines) + "\n")
    monkeypatch.setattr(bench, "TRAFFIC_FILE", stale)
    value, note = bench.read_traffic()
    assert value is None and "0000000000000000" in note
    monkeypatch.setattr(bench, "TRAFFIC_FILE", tmp_path / "absent.md")
    assert bench.read_traffic() == (None, "no counter summary")


def test_committed_traffic_summary_matches_these_sources():
    value, note = bench.read_traffic()
    assert value is not None, note
    assert 19_220_736 <= value < 2 * 19_220_736  # at least the algorithmic bytes
