"""The persistent code-object cache.  On the CPU, planning with compile=True
runs hiprtc, which is all the cache sits in front of: hits, damaged and
truncated entries, the key's compiler tag.  On the GPU, fresh child
processes fill the cache, then run the five benchmark graphs from it alone
(no hiprtc call) and match the oracle, also after an entry is damaged."""

import os
import tempfile

import pytest

import porch_amd as porch
from tests.helpers import config_graph, config_shapes, placeholder

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture
def cache_dir():
    previous = porch.disk_cache_directory()
    with tempfile.TemporaryDirectory(dir=REPO, prefix=".disk_cache_test_") as d:
        porch.set_disk_cache(d)
        porch.reset_jit_cache()
        yield d
        porch.set_disk_cache(previous or None)
        porch.reset_jit_cache()


def graph():
    return config_graph("softmax", [placeholder(s) for s in config_shapes("softmax", {"rows": 8, "cols": 256})],
                        {"rows": 8, "cols": 256})


def entries(d):
    return sorted(f for f in os.listdir(d) if f.endswith(".co"))


def test_compiled_kernels_are_stored_and_read_back(cache_dir):
    before = porch.jit_stats()
    porch.plan(graph(), compile=True)
    mid = porch.jit_stats()
    assert mid["compiles"] == before["compiles"] + 1
    assert len(entries(cache_dir)) == 1
    porch.reset_jit_cache()  # a fresh process, as far as the caches in memory go
    porch.plan(graph(), compile=True)
    after = porch.jit_stats()
    assert after["compiles"] == mid["compiles"]          # no hiprtc run
    assert after["disk_hits"] == mid["disk_hits"] + 1


def test_damaged_entries_are_recompiled_not_loaded(cache_dir):
    porch.plan(graph(), compile=True)
    (name,) = entries(cache_dir)
    path = os.path.join(cache_dir, name)
    data = bytearray(open(path, "rb").read())
    data[-1] ^= 0xFF  # flip a bit of the code: the checksum no longer matches
    open(path, "wb").write(bytes(data))
    porch.reset_jit_cache()
    before = porch.jit_stats()
    porch.plan(graph(), compile=True)
    after = porch.jit_stats()
    assert after["compiles"] == before["compiles"] + 1
    assert after["disk_hits"] == before["disk_hits"]
    # the rewritten entry is whole again
    porch.reset_jit_cache()
    porch.plan(graph(), compile=True)
    assert porch.jit_stats()["disk_hits"] == after["disk_hits"] + 1


def test_truncated_and_foreign_files_are_ignored(cache_dir):
    porch.plan(graph(), compile=True)
    (name,) = entries(cache_dir)
    path = os.path.join(cache_dir, name)
    open(path, "wb").write(open(path, "rb").read()[:40])
    porch.reset_jit_cache()
    before = porch.jit_stats()
    porch.plan(graph(), compile=True)
    assert porch.jit_stats()["compiles"] == before["compiles"] + 1


def test_each_distinct_kernel_gets_its_own_entry(cache_dir):
    porch.plan(graph(), compile=True)
    porch.plan(porch.exp(placeholder([1000])) + 1.0, compile=True)
    assert len(entries(cache_dir)) == 2


def test_cache_off_writes_nothing(cache_dir):
    porch.set_disk_cache(None)
    assert porch.disk_cache_directory() == ""
    porch.reset_jit_cache()
    porch.plan(graph(), compile=True)
    assert entries(cache_dir) == []


def test_stored_key_names_the_compiler_and_format(cache_dir):
    """The key stored in an entry ends with the hiprtc version and the
    entry format, so a different compiler or format never reads it."""
    import struct

    porch.plan(graph(), compile=True)
    (name,) = entries(cache_dir)
    data = open(os.path.join(cache_dir, name), "rb").read()
    assert data[:8] == b"PORCHCO1"
    key_size, code_size, _ = struct.unpack("<3Q", data[8:32])
    key = data[32:32 + key_size]
    assert len(data) == 32 + key_size + code_size
    tag = key[key.rindex(b"\0hiprtc "):]
    assert tag.endswith(b"\0porch code object 1")
    major, minor = tag[len(b"\0hiprtc "):-len(b"\0porch code object 1")].split(b".")
    assert int(major) >= 6 and int(minor) >= 0


# -- on the GPU: kernels read back from the cache run and give the oracle's results

def _child(directory):
    """Runs tests/disk_cache_child.py as a fresh process (never an exec of
    this one) with the cache in `directory`; its JSON report."""
    import json
    import subprocess
    import sys

    env = dict(os.environ, PORCH_CACHE_DIR=str(directory))
    result = subprocess.run([sys.executable, os.path.join(REPO, "tests", "disk_cache_child.py")],
                            capture_output=True, text=True, timeout=600, env=env, cwd=REPO)
    assert result.returncode == 0, result.stderr[-2000:]
    return json.loads(result.stdout.strip().splitlines()[-1])


@pytest.mark.gpu
def test_kernels_loaded_from_the_cache_match_the_oracle(gpu, tmp_path):
    directory = tmp_path / "cache"
    first = _child(directory)
    assert all(first["matched"].values()), first
    assert first["compiles"] == first["kernels"] and first["disk_hits"] == 0, first
    assert len(entries(directory)) == first["kernels"]

    # a fresh process: every kernel from the cache, none compiled
    second = _child(directory)
    assert all(second["matched"].values()), second
    assert second["compiles"] == 0 and second["disk_hits"] == second["kernels"], second

    # a damaged entry is compiled again (and rewritten), the rest still load
    name = entries(directory)[0]
    path = os.path.join(directory, name)
    data = bytearray(open(path, "rb").read())
    data[len(data) // 2] ^= 0x5A
    open(path, "wb").write(bytes(data))
    third = _child(directory)
    assert all(third["matched"].values()), third
    assert third["compiles"] == 1 and third["disk_hits"] == third["kernels"] - 1, third
    fourth = _child(directory)
    assert fourth["compiles"] == 0 and fourth["disk_hits"] == fourth["kernels"], fourth
