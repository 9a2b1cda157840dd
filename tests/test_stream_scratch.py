"""Ownership of the per-(device, stream) kernel scratch (split-k partial tiles,
guidance statistics), on the CPU: the rules of
seedvr2_ncnn_amd/csrc/scratch_registry.h driven over fake runtime operations
that log every call (tests/harness/scratch_harness.cpp).

  * an owner's acquire allocates and zeroes the scratch once, ordered on its
    stream, with no host wait;
  * the forward path's lookup of an owned entry makes no runtime call at all,
    and a lookup on a stream nobody owns allocates and zeroes on that stream
    without any synchronisation, and keeps the entry;
  * the last owner's release waits for that stream only, then frees;
  * entries are per (device, stream, kind).

The reference has no counterpart (ncnn's Vulkan allocators own their
workspaces); the rule replaces a device-wide synchronise that the first
split-k forward on a stream used to make."""
import ctypes
import os
import re

import pytest

from common import ROOT

HARNESS = os.path.join(ROOT, "tests", "harness", "libscratch_harness.so")
CSRC = os.path.join(ROOT, "seedvr2_ncnn_amd", "csrc")

MB64 = 64 << 20


@pytest.fixture()
def reg():
    if not os.path.exists(HARNESS):
        pytest.skip("scratch harness not built (make -C tests/harness)")
    L = ctypes.CDLL(HARNESS)
    L.hs_acquire.argtypes = [ctypes.c_int, ctypes.c_long, ctypes.c_long]
    L.hs_release.argtypes = [ctypes.c_int, ctypes.c_long]
    L.hs_get.argtypes = [ctypes.c_int, ctypes.c_long, ctypes.c_long, ctypes.POINTER(ctypes.c_long)]
    L.hs_owners.argtypes = [ctypes.c_int, ctypes.c_long]
    L.hs_take_log.argtypes = [ctypes.c_char_p, ctypes.c_int]
    L.hs_reset()
    return L


def _log(L):
    buf = ctypes.create_string_buffer(1 << 16)
    L.hs_take_log(buf, len(buf))
    return [line.split() for line in buf.value.decode().strip().split("\n") if line]


def _get(L, kind, stream, nbytes):
    out = ctypes.c_long()
    ret = L.hs_get(kind, stream, nbytes, ctypes.byref(out))
    return ret, out.value


def test_acquire_allocates_and_zeroes_on_its_stream_without_waiting(reg):
    assert reg.hs_acquire(0, 7, MB64) == 0
    log = _log(reg)
    assert [op[0] for op in log] == ["alloc", "zero"]
    assert int(log[0][2]) == MB64
    assert log[1] == ["zero", log[0][1], "7"]          # the buffer, on stream 7
    assert reg.hs_owners(0, 7) == 1


def test_forward_lookup_of_an_owned_entry_makes_no_runtime_call(reg):
    assert reg.hs_acquire(0, 7, MB64) == 0
    _log(reg)
    ret, p = _get(reg, 0, 7, MB64)
    assert ret == 0 and p != 0
    assert _log(reg) == []
    assert reg.hs_owners(0, 7) == 1


def test_release_frees_only_with_the_last_owner_after_waiting_for_that_stream(reg):
    assert reg.hs_acquire(0, 7, MB64) == 0
    assert reg.hs_acquire(0, 7, MB64) == 0
    log = _log(reg)
    assert [op[0] for op in log] == ["alloc", "zero"]   # the second owner shares it
    ptr = log[0][1]
    assert reg.hs_owners(0, 7) == 2
    assert reg.hs_release(0, 7) == 0
    assert _log(reg) == []
    assert reg.hs_release(0, 7) == 0
    assert _log(reg) == [["sync", "7", "0"], ["free", ptr, "0"]]
    assert reg.hs_owners(0, 7) == -1
    assert reg.hs_release(0, 7) == -1                   # no owner left


def test_forward_on_an_unowned_stream_makes_a_kept_entry_without_any_wait(reg):
    ret, p = _get(reg, 0, 9, MB64)
    assert ret == 0 and p != 0
    log = _log(reg)
    assert [op[0] for op in log] == ["alloc", "zero"]
    assert log[1][2] == "9"
    assert not any(op[0] == "sync" for op in log)
    assert reg.hs_owners(0, 9) == 1000                  # kept, no owner
    # an owner arriving later shares it; its release never frees it
    assert reg.hs_acquire(0, 9, MB64) == 0
    assert reg.hs_release(0, 9) == 0
    assert _log(reg) == []
    assert _get(reg, 0, 9, MB64) == (0, p)


def test_entries_are_per_stream_kind_and_device(reg):
    assert reg.hs_acquire(0, 1, MB64) == 0
    assert reg.hs_acquire(0, 2, MB64) == 0
    assert reg.hs_acquire(1, 1, 4096) == 0
    reg.hs_set_device(1)
    assert reg.hs_acquire(0, 1, MB64) == 0
    ptrs = [op[1] for op in _log(reg) if op[0] == "alloc"]
    assert len(ptrs) == 4 and len(set(ptrs)) == 4
    assert reg.hs_owners(0, 1) == 1
    reg.hs_set_device(0)
    assert reg.hs_owners(0, 1) == 1 and reg.hs_owners(1, 1) == 1 and reg.hs_owners(1, 2) == -1


def test_a_size_mismatch_and_a_failed_allocation_are_errors(reg):
    assert reg.hs_acquire(0, 1, MB64) == 0
    assert reg.hs_acquire(0, 1, MB64 // 2) == -1
    assert _get(reg, 0, 1, 1024)[0] == -1
    reg.hs_fail_alloc(1)
    assert reg.hs_acquire(0, 3, MB64) == 2
    assert reg.hs_owners(0, 3) == -1                    # nothing half-made is left
    reg.hs_fail_alloc(0)
    assert reg.hs_acquire(0, 3, MB64) == 0


def _code_lines(path):
    """Source lines without // comments."""
    out = []
    for line in open(path):
        out.append(line.split("//")[0])
    return out


def test_no_device_wide_synchronise_in_the_library():
    """No hipDeviceSynchronize anywhere in the HIP library or the layers:
    forward paths order work on streams only."""
    hits = []
    for d, _, files in os.walk(CSRC):
        for f in files:
            if f.endswith((".hip", ".cpp", ".h")):
                p = os.path.join(d, f)
                for i, line in enumerate(_code_lines(p)):
                    if re.search(r"\bhipDeviceSynchronize\b", line):
                        hits.append(f"{p}:{i + 1}")
    assert hits == []


def test_forward_scratch_lookup_never_synchronises():
    """The forward path's lookup (ScratchRegistry::get and what it calls)
    contains no synchronise call; only release does."""
    text = open(os.path.join(CSRC, "scratch_registry.h")).read()
    body = {}
    for name in ("get", "find_or_make", "release", "acquire"):
        m = re.search(r"\n    (?:int|bool) " + name + r"\([^)]*\) \{\n(.*?)\n    \}\n", text, re.S)
        assert m, name
        body[name] = m.group(1)
    assert "synchronize" not in body["get"] and "synchronize" not in body["find_or_make"]
    assert "synchronize" not in body["acquire"]
    assert "synchronize" in body["release"]
