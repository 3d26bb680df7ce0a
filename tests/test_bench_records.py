"""bench.py's recorded figures on the CPU: the comment stripper behind the source fingerprints, and
that every line of profiles/hbm_traffic.txt and profiles/kernel_counters.txt still names the code it
was measured on (bench reports a stale line as null)."""

from __future__ import annotations

import os
import re

import pytest

import bench


def test_code_only_drops_comments_and_keeps_strings():
    src = ('int a = 1; // tail\n/* block\n   comment */ const char* s = "x // y \\" z /* w */";\n\n'
           '  b();   \n#define C(x) x /* in a macro */ + 1\n')
    assert bench._code_only(src) == 'int a = 1;\n const char* s = "x // y \\" z /* w */";\n  b();\n#define C(x) x  + 1'


def test_fingerprint_ignores_comments_but_not_code(tmp_path, monkeypatch):
    csrc = tmp_path / "mote_amd" / "csrc"
    csrc.mkdir(parents=True)
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    monkeypatch.setitem(bench.KERNEL_SOURCES, "k", ["k.hip"])
    (csrc / "k.hip").write_text("// v1\n__global__ void k(int* p) { p[0] = 1; }\n")
    a = bench.source_fingerprint("k")
    (csrc / "k.hip").write_text("// v2, longer comment\n__global__ void k(int* p) { p[0] = 1; }  /* x */\n")
    assert bench.source_fingerprint("k") == a
    (csrc / "k.hip").write_text("// v2\n__global__ void k(int* p) { p[0] = 2; }\n")
    assert bench.source_fingerprint("k") != a


@pytest.mark.parametrize("name", ["hbm_traffic.txt", "kernel_counters.txt"])
def test_recorded_lines_match_the_current_sources(name):
    path = os.path.join(bench.ROOT, "profiles", name)
    lines = [ln for ln in open(path).read().splitlines() if re.match(r"^\S+ .* src=[0-9a-f]{12}$", ln)]
    assert lines
    stale = [ln for ln in lines if ln.split()[-1][4:] != bench.source_fingerprint(ln.split()[0])]
    assert not stale, f"re-collect these profiles: {stale}"
