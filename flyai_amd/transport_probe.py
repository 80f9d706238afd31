"""Loopback measurement of activation frames between two GPU buffers on one host.

    python -m flyai_amd.transport_probe [--frames 20] [--out report.json]

For each frame geometry (decode rows h[8, 4, 2880] bf16 and a 4096-token prefill chunk
h[1, 4096, 2880] bf16), a sender thread sends the activation from HBM over a loopback TCP socket
and the receiver lands it in HBM; the time is taken from the sender's first byte to the receiver's
device-ready point (stream synchronised), averaged over back-to-back frames.  Two paths:

* ``pageable``: the reference's call pattern on the same codec: ``h.cpu()`` to pageable memory,
  ``send_msg``; ``recv_msg`` into a fresh CPU tensor, then ``.to(device)``.
* ``pinned_ring``: ``send_msg`` of the device tensor (chunked D2H through the pinned ring,
  overlapped with the send) and ``recv_activation`` (chunked H2D while the next chunk arrives).

The loopback socket alone (the same bytes, CPU to CPU) is reported as the ceiling for both.
"""
import argparse
import json
import socket
import threading
import time

import torch

from . import transport as W

GEOMETRIES = {"decode_8x4": (8, 4, 2880), "prefill_1x4096": (1, 4096, 2880)}


def _loopback():
    lst = socket.socket()
    lst.bind(("127.0.0.1", 0))
    lst.listen(1)
    a = socket.create_connection(lst.getsockname(), timeout=60)
    b, _ = lst.accept()
    lst.close()
    for s in (a, b):
        W.tune_socket(s)
        s.settimeout(60)
    return a, b


def _run(path, h, frames, warmup):
    a, b = _loopback()
    dev = h.device
    n_total = frames + warmup
    marks = []

    def sender():
        for _ in range(n_total):
            if path == "pageable":
                W.send_msg(a, {"op": "verify", "h": h.cpu()})
            elif path == "pinned_ring":
                W.send_msg(a, {"op": "verify", "h": h})
            else:
                W.send_msg(a, {"op": "verify", "h": h_host})

    h_host = h.cpu()
    t = threading.Thread(target=sender, daemon=True)
    torch.cuda.synchronize()
    t.start()
    for i in range(n_total):
        if i == warmup:
            start = time.perf_counter()
        if path == "pageable":
            got = W.recv_msg(b)["h"].to(dev)
        elif path == "pinned_ring":
            got = W.recv_activation(b, dev)["h"]
        else:
            got = W.recv_msg(b)["h"]
        if path != "socket_only":
            torch.cuda.current_stream(dev).synchronize()
        marks.append(got)
        if len(marks) > 2:
            marks.pop(0)
    elapsed = time.perf_counter() - start
    t.join(60)
    ok = torch.equal(marks[-1].cpu() if marks[-1].device.type != "cpu" else marks[-1], h.cpu())
    a.close(), b.close()
    nbytes = W.frame_length({"op": "verify", "h": h})
    return {"ms_per_frame": elapsed / frames * 1e3, "GBps": nbytes * frames / elapsed / 1e9,
            "frame_bytes": nbytes, "bytes_equal": bool(ok)}


def measure(frames=20, warmup=3, device="cuda"):
    report = {"schema": "flyai-activation-wire-loopback/1", "device": torch.cuda.get_device_name(device),
              "transport": "loopback_tcp", "sock_buf": W.SOCK_BUF, "chunk_bytes": W.CHUNK_BYTES,
              "ring_slots": W.RING_SLOTS, "frames": frames, "warmup": warmup, "results": {}}
    for name, shape in GEOMETRIES.items():
        g = torch.Generator(device=device)
        g.manual_seed(0)
        h = torch.randn(shape, device=device, generator=g).to(torch.bfloat16)
        report["results"][name] = {p: _run(p, h, frames, warmup) for p in ("socket_only", "pageable", "pinned_ring")}
        print(json.dumps({name: report["results"][name]}), flush=True)
    return report


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--frames", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--out", default=None)
    args = ap.parse_args(argv)
    rep = measure(args.frames, args.warmup)
    if args.out:
        with open(args.out, "w") as f:
            json.dump(rep, f, indent=2)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
