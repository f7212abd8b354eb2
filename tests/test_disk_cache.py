"""The persistent code-object cache (no GPU: planning with compile=True runs
hiprtc, which is all the cache sits in front of)."""

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
