"""The build recipe: asca_amd/build.py compiles each HIP source with the common
flags plus its own, falls back to the common flags when a source's own flags
make the compiler fail, and INTEGRATION.md's build.rs (the reference's
rust/build.rs:12-59 counterpart) carries the same flag table.  CPU only: hipcc
cross-compiles for gfx950 without a GPU."""
import re
import shutil
from pathlib import Path

import pytest

from asca_amd import build as hb

ROOT = Path(__file__).resolve().parents[1]


def _build_rs() -> str:
    text = (ROOT / "INTEGRATION.md").read_text()
    m = re.search(r"## rust/build\.rs\s+```rust\n(.*?)```", text, re.S)
    assert m, "INTEGRATION.md has no build.rs block"
    return m.group(1)


def test_build_rs_flags_match_build_py():
    rs = _build_rs()
    m = re.search(r"const HIP_FLAGS: &\[&str\] = &\[(.*?)\];", rs, re.S)
    assert m, "build.rs declares no HIP_FLAGS"
    assert re.findall(r'"([^"]*)"', m.group(1)) == hb.HIP_FLAGS
    m = re.search(r"const EXTRA_FLAGS: .*? = &\[(.*?)\n\];", rs, re.S)
    assert m, "build.rs declares no EXTRA_FLAGS"
    rs_extra = {name: re.findall(r'"([^"]*)"', flags)
                for name, flags in re.findall(r'\("([^"]+)", &\[(.*?)\]\)', m.group(1))}
    assert rs_extra == hb.EXTRA_FLAGS
    # the per-source compile with the common-flags fallback, then one link
    assert "compile(&hipcc, &p, &inc, extra, &obj)" in rs
    assert "compile(&hipcc, &p, &inc, &[], &obj)" in rs


@pytest.mark.skipif(shutil.which(hb.hipcc()) is None and not Path(hb.hipcc()).exists(), reason="no hipcc")
def test_compile_falls_back_to_common_flags(tmp_path, monkeypatch, capsys):
    src = hb.CSRC / "util.hip"
    monkeypatch.setitem(hb.EXTRA_FLAGS, "util.hip", ["-mllvm", "-asca-no-such-option"])
    obj = tmp_path / "util.o"
    hb._compile(src, str(obj), ["-I", str(ROOT / "include")], verbose=False)
    assert obj.exists() and obj.stat().st_size > 0
    assert "compiling it with the common flags only" in capsys.readouterr().err
