"""The static library (furnace_amd/lib/libfurnace_hip.a) holds every entry
point include/*.h declares, and tests/capi_static.c, linked against it with
no libfurnace_hip.so at run time, reproduces the tiny golden model's 32
greedy ids through frn_create / frn_upload / frn_finalize / frn_prefill /
frn_decode_greedy (GPU)."""
import os
import subprocess

import pytest

import furnace_amd as fa
from furnace_amd import _build
from test_capi import declared_symbols
from test_golden import fixture, write_model


def test_archive_defines_every_declared_symbol():
    out = subprocess.run(["nm", "--defined-only", "-g", _build.STATIC], capture_output=True, text=True,
                         check=True).stdout
    defined = {line.split()[-1] for line in out.splitlines() if line.strip() and not line.endswith(":")}
    missing = sorted(declared_symbols() - defined)
    assert not missing, missing


def test_c_caller_does_not_load_the_shared_library():
    out = subprocess.run(["readelf", "-d", _build.CAPI_STATIC], capture_output=True, text=True, check=True).stdout
    needed = [l for l in out.splitlines() if "(NEEDED)" in l]
    assert needed and not any("furnace_hip" in l for l in needed), needed


@pytest.mark.gpu
def test_static_c_caller_reproduces_golden_ids(hip, tmp_path):
    f = fixture("tiny.npz")
    path = str(tmp_path / "tiny.gguf")
    write_model(f, path)
    ids = ",".join(str(int(i)) for i in f["prompt"])
    want = ",".join(str(int(i)) for i in f["ids"])
    print("capi_static on tiny.npz's model", flush=True)
    r = subprocess.run([_build.CAPI_STATIC, path, ids, want], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "32 of 32 ids match" in r.stdout
