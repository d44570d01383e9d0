"""The product path never reaches the CPU oracle: the package's sources name
nothing under oracle/, the built library links no oracle library, and the
Python loader raises when the HIP library is not built (no CPU fallback)."""
import os
import re
import subprocess

import pytest

import glacier_attn as ga

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "glacier.tune_amd")
SOURCE_EXT = (".py", ".hip", ".cpp", ".hpp", ".h")


def _package_sources():
    for base in (PKG, os.path.join(ROOT, "include")):
        for dirpath, dirnames, files in os.walk(base):
            dirnames[:] = [d for d in dirnames if not d.startswith(("_", "."))]
            for f in files:
                if f.endswith(SOURCE_EXT):
                    yield os.path.join(dirpath, f)


def test_package_sources_do_not_name_the_oracle():
    pat = re.compile(r"\boracle\b|liboracle")
    files = list(_package_sources())
    assert any(f.endswith("engine.cpp") for f in files)
    hits = []
    for path in files:
        with open(path, encoding="utf-8") as fh:
            for n, line in enumerate(fh, 1):
                if pat.search(line):
                    hits.append(f"{os.path.relpath(path, ROOT)}:{n}: {line.strip()}")
    assert not hits, "product sources reference the oracle:\n" + "\n".join(hits)


def test_library_links_no_oracle():
    if not os.path.exists(ga.LIB_PATH):
        pytest.skip("library not built")
    out = subprocess.run(["readelf", "-d", ga.LIB_PATH], capture_output=True, text=True, check=True).stdout
    needed = re.findall(r"\(NEEDED\).*\[(.+)\]", out)
    assert needed, "readelf listed no NEEDED entries"
    assert not [n for n in needed if "oracle" in n], needed


def test_loader_raises_without_the_library(monkeypatch, tmp_path):
    monkeypatch.setattr(ga, "_lib", None)
    monkeypatch.setattr(ga, "LIB_PATH", str(tmp_path / "libglacier_attn.so"))
    with pytest.raises(RuntimeError, match="not built"):
        ga.load()
