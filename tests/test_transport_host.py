"""Activation frame codec and receive pool on the CPU.

Mirrors the reference's codec tests: the hostile-frame cases of tests/test_wire_hardening.py
(oversized length, lying shapes, bad dims, dead-edge ConnectionError) and the pool cases of
tests/test_receive_buffers.py.  The byte layout is pinned by the frame the reference's own test
builds by hand (tests/test_wire_hardening.py:49-53) and by a literal frame written out below."""
import gc
import socket
import struct
import threading

import pytest
import torch

from flyai_amd import transport as W


@pytest.fixture(autouse=True)
def reset_pool():
    W.configure_receive_pool(0)
    yield
    gc.collect()
    W.configure_receive_pool(0)


def _pair():
    a, b = socket.socketpair()
    a.settimeout(5)
    b.settimeout(5)
    return a, b


def exchange(value, recv=W.recv_msg):
    left, right = _pair()
    t = threading.Thread(target=W.send_msg, args=(left, value))
    t.start()
    try:
        out = recv(right)
        t.join(5)
        assert not t.is_alive()
        return out
    finally:
        left.close()
        right.close()


def _tensor_frame(shape, blob, dtype="torch.float32"):
    """One tensor node + its blob, built the way the reference's hardening test builds it."""
    import json
    head = json.dumps({"__t__": 0, "dtype": dtype, "shape": shape}).encode()
    return struct.pack("!I", len(head)) + head + struct.pack("!Q", len(blob)) + blob


# ---- byte layout -----------------------------------------------------------------------------------

def test_single_tensor_frame_matches_hand_built_layout():
    t = torch.tensor([1.5, 2.5])
    assert W._pack(t) == _tensor_frame([2], struct.pack("<2f", 1.5, 2.5))


def test_literal_frame_bytes():
    """{"op": "verify", "h": bf16 [1, 2] = (1.0, -2.0), "start": 7}: the whole wire image."""
    msg = {"op": "verify", "h": torch.tensor([[1.0, -2.0]], dtype=torch.bfloat16), "start": 7}
    head = b'{"op": "verify", "h": {"__t__": 0, "dtype": "torch.bfloat16", "shape": [1, 2]}, "start": 7}'
    body = len(head).to_bytes(4, "big") + head + (4).to_bytes(8, "big") + bytes([0x80, 0x3F, 0x00, 0xC0])
    left, right = _pair()
    n = W.send_msg(left, msg)
    wire = right.recv(1 << 16)
    left.close(), right.close()
    assert wire == len(body).to_bytes(8, "big") + body and n == len(wire) == W.frame_length(msg)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32, torch.float8_e4m3fn,
                                   torch.float8_e5m2, torch.int64, torch.int32, torch.uint8, torch.bool])
def test_roundtrip_preserves_bytes(dtype):
    original = torch.arange(20).to(dtype).reshape(2, 10)
    got = exchange({"h": original, "ids": torch.tensor([[1, 2]]), "n": [1, (2, 3)], "f": None})
    assert got["h"].dtype == dtype and torch.equal(got["h"].view(torch.uint8), original.view(torch.uint8))
    assert got["n"] == [1, [2, 3]] and got["f"] is None


def test_legit_roundtrip_with_empty_and_scalar_tensors():
    msg = {"op": "verify", "h": torch.randn(1, 5, 8, dtype=torch.bfloat16), "start": 7, "ids": [1, 2, 3],
           "flag": True, "empty": torch.empty(0, 8), "scalar": torch.tensor(3),
           "strided": torch.arange(12.0).reshape(3, 4).t()}
    got = exchange(msg)
    assert torch.equal(got["h"], msg["h"]) and got["start"] == 7 and got["flag"] is True
    assert got["empty"].shape == (0, 8) and int(got["scalar"]) == 3
    assert torch.equal(got["strided"], msg["strided"])
    assert W._pack(got) == W._pack(msg)


def test_unencodable_values_refused():
    with pytest.raises(TypeError):
        W._pack({"x": object()})
    with pytest.raises(TypeError):
        W._pack({"x": torch.zeros(2, dtype=torch.complex64)})


# ---- hostile frames --------------------------------------------------------------------------------

def test_oversized_length_rejected_before_body():
    a, b = _pair()
    a.sendall(struct.pack("!Q", W.MAX_FRAME + 1))
    with pytest.raises(ConnectionError, match="MAX_FRAME"):
        W.recv_msg(b)
    a.close(), b.close()


def test_length_at_cap_is_accepted(monkeypatch):
    a, b = _pair()
    body = _tensor_frame([2], struct.pack("<2f", 1.5, 2.5))
    monkeypatch.setattr(W, "MAX_FRAME", len(body))
    a.sendall(struct.pack("!Q", len(body)) + body)
    assert torch.equal(W.recv_msg(b), torch.tensor([1.5, 2.5]))
    a.close(), b.close()


def test_empty_blob_huge_shape_rejected():
    with pytest.raises(ValueError):
        W._unpack(_tensor_frame([100_000_000], b""))


@pytest.mark.parametrize("shape,blob", [([100], b"\0" * 8), ([1], b"\0" * 400), ([2, 3], b"\0" * 8)])
def test_shape_blob_size_mismatch_rejected(shape, blob):
    with pytest.raises(ValueError):
        W._unpack(_tensor_frame(shape, blob))


@pytest.mark.parametrize("shape", [[-1], [2, -3], [1.5], ["x"], [1] * 33])
def test_bad_dim_rejected(shape):
    with pytest.raises(ValueError):
        W._unpack(_tensor_frame(shape, b""))


@pytest.mark.parametrize("body", [b"", struct.pack("!I", 999), struct.pack("!I", 2) + b"{}" + b"short",
                                  struct.pack("!I", 2) + b"{}" + struct.pack("!Q", 99),
                                  _tensor_frame([100_000_000], b""), _tensor_frame([2], b"\0" * 8, "torch.cfloat"),
                                  struct.pack("!I", 3) + b"{x}"])
def test_recv_msg_turns_malformed_frames_into_dead_edges(body):
    W.configure_receive_pool(8192)
    a, b = _pair()
    a.sendall(struct.pack("!Q", len(body)) + body)
    with pytest.raises(ConnectionError, match="malformed"):
        W.recv_msg(b)
    a.close(), b.close()
    gc.collect()
    assert W.receive_pool_status()["live_slots"] == 0


def test_peer_close_mid_frame_is_connection_error():
    a, b = _pair()
    a.sendall(struct.pack("!Q", 100) + b"\0" * 10)
    a.close()
    with pytest.raises(ConnectionError, match="closed"):
        W.recv_msg(b)
    b.close()


# ---- receive pool ----------------------------------------------------------------------------------

def test_pooled_view_keeps_its_slot_until_last_view_dies():
    W.configure_receive_pool(8192, slots=1)
    original = torch.arange(20).to(torch.bfloat16).reshape(2, 10)
    msg = exchange({"h": original, "ids": torch.tensor([[1, 2]])})
    view = msg["h"].reshape(-1)[3:9]
    expected = view.clone()
    del msg
    assert W.receive_pool_status()["live_slots"] == 1
    other = exchange({"h": torch.full((20,), 77.0)})       # slot busy: owned-frame fallback
    assert torch.equal(view, expected) and W.receive_pool_status()["fallback_frames"] == 1
    del view, other
    assert W.receive_pool_status()["live_slots"] == 0
    again = exchange({"h": original})
    assert W.receive_pool_status()["borrowed_frames"] == 2 and torch.equal(again["h"], original)


def test_pooled_frames_have_independent_storage_and_slots_are_reused():
    W.configure_receive_pool(8192, slots=2)
    first = exchange({"h": torch.arange(40)})
    ptr = first["h"].data_ptr()
    second = exchange({"h": torch.arange(40) + 10})
    assert first["h"].data_ptr() != second["h"].data_ptr() and torch.equal(first["h"], torch.arange(40))
    del first
    third = exchange({"h": torch.arange(40) + 20})
    assert third["h"].data_ptr() == ptr and torch.equal(third["h"], torch.arange(40) + 20)


def test_reconfigure_refused_while_views_live():
    W.configure_receive_pool(8192)
    held = exchange({"h": torch.ones(32)})
    with pytest.raises(RuntimeError, match="views of pooled frames are live"):
        W.configure_receive_pool(0)
    del held


def test_control_frame_releases_pool():
    W.configure_receive_pool(8192)
    assert exchange({"op": "reset", "job_id": "new", "nonce": "a" * 64})["op"] == "reset"
    assert W.receive_pool_status()["live_slots"] == 0


def test_budget_counts_resize_peak_and_busy_slots():
    pool = W.ReceiveBufferPool(2048, slots=2)
    first, second = pool.borrow(100), pool.borrow(900)
    assert pool.borrow(100) is None
    del first, second
    assert pool.borrow(1800) is None          # old 2 x 1 KiB + a 2 KiB replacement exceeds the budget
    assert pool.snapshot()["allocated_bytes"] <= 2048


def test_pool_limits_and_exhaustion_fallback():
    for bad in (dict(budget_bytes=100), dict(budget_bytes=1 << 30), dict(budget_bytes=4096, slots=0)):
        with pytest.raises(ValueError):
            W.ReceiveBufferPool(**bad)
    W.configure_receive_pool(1024, slots=1)
    got = exchange({"h": torch.arange(8192)})
    assert got["h"].shape == (8192,) and W.receive_pool_status()["fallback_frames"] == 1
    assert W.receive_pool_status()["allocated_bytes"] == 0


def test_pool_release_needs_no_cyclic_gc():
    W.configure_receive_pool(8192, slots=1)
    was = gc.isenabled()
    gc.disable()
    try:
        for _ in range(10):
            got = exchange({"h": torch.arange(20)})
            assert W._pack(got) == W._pack({"h": torch.arange(20)})
            del got
            assert W.receive_pool_status()["live_slots"] == 0
        assert W.receive_pool_status()["fallback_frames"] == 0
    finally:
        if was:
            gc.enable()


# ---- asynchronous sender ---------------------------------------------------------------------------

def test_async_sender_fifo_and_error_surfaces_on_next_put():
    a, b = _pair()
    sender = W.AsyncSender(a)
    for i in range(5):
        sender.put({"i": i, "h": torch.full((3,), float(i))})
    got = [W.recv_msg(b) for _ in range(5)]
    assert [g["i"] for g in got] == list(range(5)) and torch.equal(got[4]["h"], torch.full((3,), 4.0))
    b.close()
    sender.put({"h": torch.zeros(1 << 20)})        # fails in the background: peer is gone
    sender.thread.join(0.5)
    for _ in range(50):
        if sender.error is not None:
            break
        threading.Event().wait(0.05)
    with pytest.raises(OSError):
        sender.put({"i": 99})
    sender.close()
    sender.close()
    assert not sender.thread.is_alive()
    with pytest.raises(RuntimeError, match="closed"):
        sender.put({"i": 100})
