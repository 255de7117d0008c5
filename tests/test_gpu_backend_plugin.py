"""The backend-amd-hip plugin on a gfx950 device: a model plugin's whole
resource lifecycle through the four device contracts, as the reference's
DeepSeek and Qwen plugins drive backend-nvidia-cuda (prepare the device,
allocate device and pinned memory, upload weights, retain and bind the
device context, create a stream and an event, copy and fill asynchronously,
record/query/synchronize, then release everything and drain).

Bytes moved by copies and the fill kernel are checked exactly against a
numpy model of the buffers.
"""
import ctypes as C

import numpy as np
import pytest

from pih_amd import backend as B
from pih_amd.abi import FAILED_PRECONDITION, INVALID_ARGUMENT, OK

pytestmark = pytest.mark.gpu

MIB = 1 << 20


@pytest.fixture(scope="module")
def dev():
    host = B.PluginHost().load().activate()
    yield B.Device(host)


def _ok(st):
    assert st.code == OK, st


def test_full_resource_lifecycle(dev):
    d = dev
    assert d.prepare(0, 8, 9).code == FAILED_PRECONDITION  # not gfx950
    _ok(d.prepare(0, 9, 5))
    _ok(d.prepare(0, 9, 5))  # idempotent
    assert d.prepare(0, 9, 4).code == FAILED_PRECONDITION

    st, a = d.allocate(0, MIB, alignment=128)
    _ok(st)
    assert a.address % 256 == 0 and a.bytes == MIB and a.alignment == 256 and a.generation > 0
    assert (a.device_ordinal, a.memory_kind) == (0, B.MEMORY_DEVICE)
    st, b = d.allocate(0, MIB)
    _ok(st)
    st, z = d.allocate(0, 0)
    _ok(st)
    assert z.address == 0 and z.generation > b.generation
    _ok(d.deallocate(z))
    st, p = d.allocate(-1, MIB, pinned=True)
    _ok(st)
    assert p.memory_kind == B.MEMORY_PINNED_HOST and p.address % 256 == 0

    # synchronous upload into the owned range only
    rng = np.random.default_rng(7)
    pattern = rng.integers(0, 256, MIB, dtype=np.uint8)
    _ok(d.copy_h2d(0, a.address, pattern.ctypes.data, MIB))
    assert d.copy_h2d(0, a.address + 16, pattern.ctypes.data, MIB).code == FAILED_PRECONDITION
    # a range running past the end of `a` (even into a neighbouring allocation) is not owned
    assert d.copy_h2d(0, a.address + MIB - 8, pattern.ctypes.data, 16).code == FAILED_PRECONDITION

    st, tok = d.retain(0)
    _ok(st)
    st, tok2 = d.retain(0)
    _ok(st)
    assert tok == tok2 and tok
    assert d.retain(0, flags=B.CONTEXT_SCHED_YIELD)[0].code == FAILED_PRECONDITION  # flags differ
    _ok(d.bind(0, tok))
    _ok(d.activate(tok))
    st, stream = d.create_stream(tok)
    _ok(st)
    st, event = d.create_event(tok)
    _ok(st)

    # fill an unaligned range of a, copy a -> b, b -> pinned
    off, count = 3, MIB - 11
    _ok(d.memset_async(tok, a.address + off, 0xAB, count, stream))
    _ok(d.copy_async(tok, b.address, a.address, MIB, B.COPY_D2D, stream))
    _ok(d.copy_async(tok, p.address, b.address, MIB, B.COPY_D2H, stream))
    _ok(d.record(tok, event, stream))
    _ok(d.synchronize(tok, stream))
    st, status = d.query(tok, event)
    _ok(st)
    assert status == B.EVENT_COMPLETE
    want = pattern.copy()
    want[off:off + count] = 0xAB
    got = np.frombuffer(C.string_at(p.address, MIB), dtype=np.uint8)
    assert np.array_equal(got, want)

    # pinned -> device round trip of a small pattern
    small = rng.integers(0, 256, 4096, dtype=np.uint8)
    C.memmove(p.address, small.ctypes.data, 4096)
    _ok(d.copy_async(tok, a.address + 256, p.address, 4096, B.COPY_H2D, stream))
    _ok(d.synchronize(tok, stream))
    C.memset(p.address, 0, MIB)
    _ok(d.copy_async(tok, p.address, a.address, MIB, B.COPY_D2H, stream))
    _ok(d.synchronize(tok, stream))
    want[256:256 + 4096] = small
    assert np.array_equal(np.frombuffer(C.string_at(p.address, MIB), dtype=np.uint8), want)

    # ownership: pageable host memory, device memory as "pinned", out-of-range ranges
    _ok(d.validate_pinned(tok, p.address + 100))
    assert d.validate_pinned(tok, a.address).code == FAILED_PRECONDITION
    assert d.validate_pinned(tok, pattern.ctypes.data).code == FAILED_PRECONDITION
    assert d.copy_async(tok, a.address, pattern.ctypes.data, 64, B.COPY_H2D, stream).code == FAILED_PRECONDITION
    assert d.copy_async(tok, b.address + 8, a.address, MIB, B.COPY_D2D, stream).code == FAILED_PRECONDITION
    assert d.memset_async(tok, p.address, 1, 16, stream).code == FAILED_PRECONDITION  # fills are device-only
    assert d.copy_async(tok, a.address, b.address, 64, 7, stream).code == INVALID_ARGUMENT
    _ok(d.clean_last_error(tok))

    # teardown order: live resources block release and drain
    assert d.release(0, tok).code == FAILED_PRECONDITION
    assert d.host.phase("drain").code == FAILED_PRECONDITION
    _ok(d.destroy_event(event))
    assert d.destroy_event(event).code == FAILED_PRECONDITION
    _ok(d.destroy_stream(stream))
    _ok(d.release(0, tok))
    _ok(d.release(0, tok2))
    assert d.release(0, tok).code == FAILED_PRECONDITION
    stale = B.Allocation.from_buffer_copy(a)
    stale.generation += 1
    assert d.deallocate(stale).code == FAILED_PRECONDITION
    assert d.deallocate(p).code == INVALID_ARGUMENT  # pinned record through the device call
    _ok(d.deallocate(a))
    _ok(d.deallocate(b))
    _ok(d.deallocate(p, pinned=True))
    assert d.deallocate(a).code == FAILED_PRECONDITION
    d.host.shutdown()
