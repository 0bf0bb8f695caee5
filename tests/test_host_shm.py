"""CPU tests of the shared CPU cache slabs (POSIX shm), the entry points of
csrc/common/mem_alloc.cpp:252-410: a creator and its peers, here a child
process, see one another's writes; names are exclusive; failures unlink
what they created; a read-only peer cannot write; a NUMA interleave is a
policy of the slab itself.  Attach failures keep the reference's
"shm_open attach failed" text (tests/v1/test_shared_slab_startup.py:40-41).
No GPU call is made."""

import ctypes
import os
import subprocess
import sys
import uuid

import pytest

from lmcache_amd import c_ops

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture
def name():
    n = f"/lmc_test_{os.getpid()}_{uuid.uuid4().hex[:8]}"
    yield n
    c_ops.unlink_shm(n)


def _buf(ptr, size):
    return (ctypes.c_ubyte * size).from_address(ptr)


def test_create_attach_share_and_free(name):
    size = 3 * 4096 + 100
    p = c_ops.alloc_shm_pinned_ptr(size, name)
    b = _buf(p, size)
    assert bytes(b) == bytes(size)  # fresh segment reads zero
    b[0], b[size - 1] = 17, 99
    q = c_ops.attach_shm_pinned_ptr(size, name)
    assert q != p
    qb = _buf(q, size)
    assert qb[0] == 17 and qb[size - 1] == 99
    qb[5000] = 7
    assert b[5000] == 7
    c_ops.detach_shm_pinned_ptr(q, size)
    c_ops.free_shm_pinned_ptr(p, size, name)
    with pytest.raises(RuntimeError, match="cannot open shared-memory segment"):
        c_ops.attach_shm_pinned_ptr(size, name)


def test_peer_process_sees_and_writes(name):
    size = 1 << 20
    p = c_ops.alloc_shm_pinned_ptr(size, name)
    b = _buf(p, size)
    for i in range(0, size, 65536):
        b[i] = (i >> 16) & 0xFF
    child = f"""
import ctypes, sys
sys.path[:0] = [{REPO!r}, {os.path.join(REPO, 'lmcache-ascend_amd')!r}]
from lmcache_amd import c_ops
q = c_ops.attach_shm_pinned_ptr({size}, {name!r})
b = (ctypes.c_ubyte * {size}).from_address(q)
assert all(b[i] == ((i >> 16) & 0xFF) for i in range(0, {size}, 65536))
b[{size} - 1] = 0xAB
c_ops.detach_shm_pinned_ptr(q, {size})
print("ok")
"""
    res = subprocess.run([sys.executable, "-c", child], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    assert res.stdout.strip() == "ok"
    assert b[size - 1] == 0xAB
    c_ops.free_shm_pinned_ptr(p, size, name)


def test_read_only_peer_cannot_write(name):
    size = 8192
    p = c_ops.alloc_shm_pinned_ptr(size, name)
    _buf(p, size)[100] = 5
    child = f"""
import ctypes, sys
sys.path[:0] = [{REPO!r}, {os.path.join(REPO, 'lmcache-ascend_amd')!r}]
from lmcache_amd import c_ops
q = c_ops.attach_shm_pinned_ptr({size}, {name!r}, writable=False)
b = (ctypes.c_ubyte * {size}).from_address(q)
print(b[100], flush=True)
b[100] = 1
print("wrote")
"""
    res = subprocess.run([sys.executable, "-c", child], capture_output=True, text=True, timeout=120)
    assert res.stdout.splitlines()[0] == "5"
    assert res.returncode == -11 and "wrote" not in res.stdout  # SIGSEGV on the write
    assert _buf(p, size)[100] == 5
    c_ops.free_shm_pinned_ptr(p, size, name)


def test_duplicate_name_is_refused(name):
    p = c_ops.alloc_shm_pinned_ptr(4096, name)
    with pytest.raises(RuntimeError, match="the name is taken"):
        c_ops.alloc_shm_pinned_ptr(4096, name)
    c_ops.free_shm_pinned_ptr(p, 4096, name)
    p = c_ops.alloc_shm_pinned_ptr(4096, name)  # the name is free again
    c_ops.free_shm_pinned_ptr(p, 4096, name)


def test_argument_errors(name):
    with pytest.raises(RuntimeError, match="alloc_shm_pinned_ptr: size must be positive"):
        c_ops.alloc_shm_pinned_ptr(0, name)
    with pytest.raises(RuntimeError, match="a slab name is required"):
        c_ops.alloc_shm_pinned_ptr(4096, "")
    with pytest.raises(RuntimeError, match="attach_shm_pinned_ptr: size must be positive"):
        c_ops.attach_shm_pinned_ptr(0, name)
    with pytest.raises(RuntimeError, match="free_shm_pinned_ptr: the slab pointer is null"):
        c_ops.free_shm_pinned_ptr(0, 4096, name)
    with pytest.raises(RuntimeError, match="detach_shm_pinned_ptr: size must be positive"):
        c_ops.detach_shm_pinned_ptr(4096, 0)
    with pytest.raises(RuntimeError, match="not a valid node id"):
        c_ops.alloc_shm_pinned_ptr(4096, name, [-1])
    with pytest.raises(RuntimeError, match="cannot open shared-memory segment"):
        c_ops.attach_shm_pinned_ptr(4096, name)


def test_attach_beyond_segment_is_refused(name):
    p = c_ops.alloc_shm_pinned_ptr(4096, name)
    with pytest.raises(RuntimeError, match="fewer than the"):
        c_ops.attach_shm_pinned_ptr(8192, name)
    c_ops.free_shm_pinned_ptr(p, 4096, name)


def test_failed_reservation_unlinks(name):
    # larger than any /dev/shm: the reservation fails before a page is
    # touched, and the half-made segment is removed
    with pytest.raises(RuntimeError, match="cannot reserve"):
        c_ops.alloc_shm_pinned_ptr(1 << 50, name)
    with pytest.raises(RuntimeError, match="cannot open shared-memory segment"):
        c_ops.attach_shm_pinned_ptr(4096, name)


def test_unlink_missing_name_is_not_an_error(name):
    c_ops.unlink_shm(name)
    c_ops.unlink_shm(name)


def _numa_maps_line(addr):
    with open("/proc/self/numa_maps") as f:
        for line in f:
            if int(line.split()[0], 16) == addr:
                return line
    return None


def test_interleave_over_node_zero(name):
    # node 0 exists on every Linux host; the interleave is a policy of the
    # slab object, shown on the creator's mapping, and the slab reads zero
    size = 1 << 16
    p = c_ops.alloc_shm_pinned_ptr(size, name, [0])
    assert _buf(p, size)[12345] == 0
    line = _numa_maps_line(p)
    if line is not None:  # numa_maps exists on NUMA-enabled kernels
        assert "interleave" in line.split()[1], line
    n2 = name + "b"
    q = c_ops.alloc_shm_pinned_ptr(4096, n2)
    line = _numa_maps_line(q)
    if line is not None:
        assert "interleave" not in line.split()[1], line
    c_ops.free_shm_pinned_ptr(q, 4096, n2)
    c_ops.free_shm_pinned_ptr(p, size, name)


def test_bad_node_id_creates_nothing(name):
    with pytest.raises(RuntimeError, match="not a valid node id"):
        c_ops.alloc_shm_pinned_ptr(4096, name, [4096])
    with pytest.raises(RuntimeError, match="cannot open shared-memory segment"):
        c_ops.attach_shm_pinned_ptr(4096, name)
