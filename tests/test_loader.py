"""The loader's contract, as the reference's core/tests/test_kernels_prebuilt.py:13-83 states it
for its own build: a build is loaded only where its stamp is this tree's and names this GPU;
anything else is refused, never built around; the torch paths are taken by choice alone."""

import json
import shutil

import pytest

from everserve_amd import build, kernels


def test_the_stamp_is_the_sources_by_content(tmp_path, monkeypatch):
    s = kernels.stamp()
    assert set(s) == {"sources"} and len(s["sources"]) == 64
    copied = tmp_path / "csrc"
    copied.mkdir()
    for f in build.source_files():
        (copied / f.name).write_bytes(f.read_bytes())
    monkeypatch.setattr(build, "source_files",
                        lambda: [copied / f.name for f in
                                 [build.CSRC / x for x in build.SOURCES + build.HEADERS] +
                                 [build.INCLUDE / x for x in build.PUBLIC_HEADERS]])
    assert kernels.stamp() == s  # the same sources, the same stamp
    (copied / "rows.hip").write_bytes((copied / "rows.hip").read_bytes() + b"\n// changed\n")
    assert kernels.stamp()["sources"] != s["sources"]


def test_a_named_prebuilt_that_cannot_be_loaded_is_refused(tmp_path, monkeypatch):
    monkeypatch.setenv(kernels.PREBUILT_ENV, str(tmp_path))
    with pytest.raises(kernels.KernelsUnavailable, match="no usable stamp"):
        kernels._prebuilt()
    (tmp_path / kernels.STAMP).write_text(json.dumps({"sources": "0" * 64, "archs": "gfx950"}))
    with pytest.raises(kernels.KernelsUnavailable, match="built against"):
        kernels._prebuilt()
    (tmp_path / kernels.STAMP).write_text(json.dumps({**kernels.stamp(), "archs": "gfx942"}))
    monkeypatch.setattr(kernels, "device_arch", lambda: "gfx950")
    with pytest.raises(kernels.KernelsUnavailable, match="this GPU is gfx950"):
        kernels._prebuilt()
    monkeypatch.setattr(kernels, "device_arch", lambda: "gfx942")
    with pytest.raises(kernels.KernelsUnavailable, match="no libeverserve_mi355x.so"):
        kernels._prebuilt()
    monkeypatch.delenv(kernels.PREBUILT_ENV)
    assert kernels._prebuilt() is None


def test_a_prebuilt_with_our_stamp_loads(tmp_path, monkeypatch):
    for name in (kernels.LIBRARY, kernels.STAMP):
        shutil.copy(kernels._PACKAGE / name, tmp_path / name)
    monkeypatch.setenv(kernels.PREBUILT_ENV, str(tmp_path))
    monkeypatch.setattr(kernels, "device_arch", lambda: "gfx950")
    assert kernels.library_path() == tmp_path / kernels.LIBRARY
    lib = kernels.open_library(kernels.library_path())
    assert hasattr(lib, "evs_gather_rows")


def test_the_torch_paths_are_taken_by_choice_alone(monkeypatch):
    kernels.available.cache_clear()
    monkeypatch.setenv(kernels.PATHS_ENV, "torch")
    assert kernels.available() is False
    kernels.available.cache_clear()


def test_without_a_gpu_the_kernels_do_not_load():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    kernels.load.cache_clear()
    with pytest.raises(kernels.KernelsUnavailable, match="GPU"):
        kernels.load()


def test_a_build_names_the_gpus_it_runs_on():
    assert kernels.built_archs("gfx942;gfx950") == {"gfx942", "gfx950"}
    assert kernels.built_archs("gfx950:sramecc+:xnack- gfx942") == {"gfx950", "gfx942"}
