"""Activation frames from and into GPU memory through the pinned rings.  The wire image of a GPU
tensor must be byte-identical to the frame of the same tensor on the CPU (the reference's codec
reads it), and a received frame must land on the GPU unchanged, for sizes below, at and above
several ring chunks, strided sources, back-to-back frames and the asynchronous sender."""
import socket
import struct
import threading

import pytest
import torch

from flyai_amd import transport as W

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _pair():
    a, b = socket.socketpair()
    a.settimeout(30)
    b.settimeout(30)
    return a, b


def _read_n(sock, n, out):
    buf = bytearray(n)
    W._recv_into(sock, memoryview(buf))
    out.append(bytes(buf))


def _gen(seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    return g


def _cpu_frame(msg):
    cpu = {k: (v.cpu() if torch.is_tensor(v) else v) for k, v in msg.items()}
    body = W._pack(cpu)
    return struct.pack("!Q", len(body)) + body


SHAPES = [(1, 4096, 2880), (3, 5, 2880), (1, 1, 2880), (0, 2880), (2, W.CHUNK_BYTES // 2 + 17)]


@pytest.mark.parametrize("shape", SHAPES)
def test_device_send_is_byte_identical_to_cpu_frame(shape):
    print(f"device send shape={shape}", flush=True)
    h = torch.randn(shape, device=DEV, generator=_gen(1)).to(torch.bfloat16)
    msg = {"op": "verify", "h": h, "ids": torch.arange(4).reshape(1, 4), "start": 7,
           "mask": torch.ones(3, device=DEV, dtype=torch.bool)}
    want = _cpu_frame(msg)
    a, b = _pair()
    got = []
    t = threading.Thread(target=_read_n, args=(b, len(want), got))
    t.start()
    n = W.send_msg(a, msg)
    t.join(30)
    a.close(), b.close()
    assert n == len(want) == W.frame_length(msg) and got[0] == want


def test_strided_device_source_sent_in_logical_order():
    base = torch.randn(2880, 64, device=DEV, generator=_gen(2)).to(torch.bfloat16)
    msg = {"h": base.t()}
    want = _cpu_frame(msg)
    a, b = _pair()
    got = []
    t = threading.Thread(target=_read_n, args=(b, len(want), got))
    t.start()
    W.send_msg(a, msg)
    t.join(30)
    a.close(), b.close()
    assert got[0] == want


@pytest.mark.parametrize("from_device", [False, True])
def test_recv_activation_lands_on_device(from_device):
    print(f"recv_activation from_device={from_device}", flush=True)
    a, b = _pair()
    sent = []
    for i, shape in enumerate(SHAPES + [(1, 4096, 2880)]):
        h = torch.randn(shape, device=DEV, generator=_gen(10 + i)).to(torch.bfloat16)
        msg = {"op": "verify", "i": i, "h": h if from_device else h.cpu(), "ids": torch.arange(i + 1),
               "aux": [torch.tensor(float(i)), {"x": None}]}
        sent.append(msg)
    t = threading.Thread(target=lambda: [W.send_msg(a, m) for m in sent])
    t.start()
    for m in sent:
        got = W.recv_activation(b, DEV)
        assert got["op"] == "verify" and got["i"] == m["i"] and got["aux"][1] == {"x": None}
        assert got["h"].device.type == "cuda" and got["ids"].device.type == "cuda"
        assert got["h"].shape == m["h"].shape and torch.equal(got["h"].cpu(), m["h"].cpu())
        assert torch.equal(got["ids"].cpu(), m["ids"]) and float(got["aux"][0]) == m["i"]
    t.join(30)
    a.close(), b.close()


def test_recv_activation_skips_unreferenced_blobs_and_refuses_malformed():
    import json
    head = json.dumps({"h": {"__t__": 1, "dtype": "torch.float32", "shape": [2]}}).encode()
    body = (struct.pack("!I", len(head)) + head + struct.pack("!Q", 3) + b"xyz"
            + struct.pack("!Q", 8) + struct.pack("<2f", 1.5, -2.0))
    a, b = _pair()
    a.sendall(struct.pack("!Q", len(body)) + body)
    got = W.recv_activation(b, DEV)
    assert torch.equal(got["h"].cpu(), torch.tensor([1.5, -2.0]))
    for bad in (struct.pack("!I", 2) + b"{}" + struct.pack("!Q", 99),
                struct.pack("!I", len(head)) + head + struct.pack("!Q", 0),  # blob 1 missing
                struct.pack("!I", 8) + b'{"h": [}'):
        a.sendall(struct.pack("!Q", len(bad)) + bad)
        with pytest.raises(ConnectionError, match="malformed"):
            W.recv_activation(b, DEV)
    a.close(), b.close()


def test_async_sender_snapshots_device_tensors():
    a, b = _pair()
    sender = W.AsyncSender(a)
    h = torch.randn(1, 4096, 2880, device=DEV, generator=_gen(3)).to(torch.bfloat16)
    want = [h.clone()]
    sender.put({"h": h})
    h.fill_(0)                                # the caller reuses its buffer at once
    for i in range(3):
        h.add_(1)
        want.append(h.clone())
        sender.put({"h": h, "i": i})
    for w in want:
        got = W.recv_activation(b, DEV)
        torch.cuda.synchronize()
        assert torch.equal(got["h"], w)
    sender.close()
    b.close()


def test_pinned_pool_tensor_copies_to_device():
    W.configure_receive_pool(8192, pinned=True)
    try:
        a, b = _pair()
        W.send_msg(a, {"h": torch.arange(40).bfloat16()})
        got = W.recv_msg(b)
        assert got["h"].is_pinned()
        dev = got["h"].to(DEV, non_blocking=True)
        torch.cuda.synchronize()
        assert torch.equal(dev.cpu(), torch.arange(40).bfloat16())
        a.close(), b.close()
        del got
    finally:
        import gc
        gc.collect()
        W.configure_receive_pool(0)
