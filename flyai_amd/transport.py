"""Inter-stage activation frames, with device-resident activations moved through pinned host memory.

Frame format (the reference's engine wire, ``shard/transport.py:85-111`` and ``:190-224``; it must
stay byte-identical so either end can be this module or the reference's):

    u64be  n                       length of the body that follows (refused above MAX_FRAME)
    u32be  hlen, hlen bytes        JSON header (json.dumps defaults); a tensor is the node
                                   {"__t__": index, "dtype": "torch.bfloat16", "shape": [...]}
    repeat: u64be blen, blen bytes the raw little-endian bytes of tensor `index`, in index order

A tensor's declared shape times its element size must equal its blob length, and anything that
does not parse is a dead edge: ``recv_msg`` raises ConnectionError, never an unbounded allocation.

What is different here is where the bytes go.  The reference copies a GPU activation to pageable
host memory (``.cpu()``), sends it, and on the far side copies the frame into a fresh CPU tensor
and from there to the GPU.  Here a GPU tensor in a message is copied in chunks into a small ring of
pinned host buffers on a copy stream, and each chunk goes to the socket as soon as its copy event
fires, so the D2H copy overlaps the send; ``recv_activation`` reads each chunk into a pinned ring
slot and starts its H2D copy straight into the destination device tensor while the next chunk is
still arriving.  No frame-sized host buffer exists on either side of the device path.
"""
import ctypes
import json
import os
import queue
import socket
import struct
import threading
import weakref

import numpy as np
import torch

_DTYPES = {str(d): d for d in (torch.float32, torch.float16, torch.bfloat16, torch.float8_e4m3fn,
                               torch.float8_e5m2, torch.int64, torch.int32, torch.uint8, torch.bool)}
_ITEMSIZE = {d: torch.empty(0, dtype=d).element_size() for d in _DTYPES.values()}

# Largest body a receiver accepts; the length prefix is read before anything authenticates the
# frame, so a larger claim is refused before the body is read (env M25_MAX_FRAME, bytes).
MAX_FRAME = int(os.environ.get("M25_MAX_FRAME") or 256 * 1024 * 1024)
SOCK_BUF = 32 << 20          # socket buffers sized for a prefill-chunk activation in flight
CHUNK_BYTES = 4 << 20        # device <-> pinned copy granularity of the device path
RING_SLOTS = 4               # pinned ring depth per direction
_IOV_MAX = 512               # segments per sendmsg call (below the kernel's UIO_MAXIOV)


# ---- header ----------------------------------------------------------------------------------------

def _encode(o, leaves):
    if torch.is_tensor(o):
        if o.dtype not in _ITEMSIZE:
            raise TypeError(f"transport cannot encode tensor dtype {o.dtype}")
        leaves.append(o.detach())
        return {"__t__": len(leaves) - 1, "dtype": str(o.dtype), "shape": list(o.shape)}
    if isinstance(o, dict):
        return {k: _encode(v, leaves) for k, v in o.items()}
    if isinstance(o, (list, tuple)):
        return [_encode(v, leaves) for v in o]
    if o is None or isinstance(o, (bool, int, float, str)):
        return o
    raise TypeError(f"transport cannot encode {type(o).__name__}")


def _header(obj):
    """(header bytes, tensor leaves in index order).  Reads shapes and dtypes only, no data.
    Module-level recursion (no self-referencing closure) so no reference cycle holds the leaves."""
    leaves = []
    return json.dumps(_encode(obj, leaves)).encode(), leaves


def _nbytes(t):
    return t.numel() * _ITEMSIZE[t.dtype]


def frame_length(obj):
    """Bytes one message occupies on the wire, length prefix included (no data is touched)."""
    head, leaves = _header(obj)
    return 8 + 4 + len(head) + sum(8 + _nbytes(t) for t in leaves)


def _host_bytes(t):
    """A uint8 view of a CPU tensor's data (made contiguous first)."""
    t = t.contiguous()
    return memoryview(t.reshape(-1).view(torch.uint8).numpy())


def _pack_parts(obj):
    """The body of a message with only CPU tensors, as a list of segments (no concatenation)."""
    head, leaves = _header(obj)
    parts = [struct.pack("!I", len(head)) + head]
    for t in leaves:
        if t.device.type != "cpu":
            t = t.cpu()
        parts.append(struct.pack("!Q", _nbytes(t)))
        parts.append(_host_bytes(t))
    return parts


def _pack(obj) -> bytes:
    return b"".join(bytes(p) for p in _pack_parts(obj))


# ---- decode ----------------------------------------------------------------------------------------

def _tensor_spec(node, n_blobs=None):
    """(dtype, shape, nbytes, index) of a tensor node, validated; ValueError if malformed."""
    dt = _DTYPES.get(node.get("dtype"))
    if dt is None:
        raise ValueError(f"unknown tensor dtype {node.get('dtype')!r}")
    index = node["__t__"]
    if type(index) is not int or index < 0 or (n_blobs is not None and index >= n_blobs):
        raise ValueError("invalid tensor blob index")
    shape = node.get("shape")
    if not isinstance(shape, list) or len(shape) > 32:
        raise ValueError("invalid tensor shape")
    numel = 1
    for d in shape:
        if type(d) is not int or d < 0:
            raise ValueError(f"bad tensor dim {d!r}")
        numel *= d
    return dt, shape, numel * _ITEMSIZE[dt], index


def _decode(node, make_tensor):
    if isinstance(node, dict):
        if "__t__" in node:
            return make_tensor(node)
        return {k: _decode(v, make_tensor) for k, v in node.items()}
    if isinstance(node, list):
        return [_decode(v, make_tensor) for v in node]
    return node


def _split_body(mv):
    """(header object, blob memoryviews) of a frame body."""
    if len(mv) < 4:
        raise ValueError("truncated frame header")
    (hlen,) = struct.unpack_from("!I", mv, 0)
    if hlen > len(mv) - 4:
        raise ValueError("header length exceeds frame")
    head = json.loads(bytes(mv[4:4 + hlen]))
    blobs, off = [], 4 + hlen
    while off < len(mv):
        if len(mv) - off < 8:
            raise ValueError("truncated blob length")
        (blen,) = struct.unpack_from("!Q", mv, off)
        off += 8
        if blen > len(mv) - off:
            raise ValueError("blob length exceeds frame")
        blobs.append(mv[off:off + blen])
        off += blen
    return head, blobs


def _unpack(buf, *, copy_tensors=True):
    """Decode one frame body into CPU tensors; ValueError if it is malformed.  With
    copy_tensors=False the tensors view `buf` (which must then outlive them)."""
    head, blobs = _split_body(memoryview(buf))

    def make(node):
        dt, shape, nbytes, index = _tensor_spec(node, len(blobs))
        blob = blobs[index]
        if nbytes != len(blob):
            raise ValueError(f"tensor {shape} needs {nbytes} bytes, blob has {len(blob)}")
        if nbytes == 0:
            return torch.empty(shape, dtype=dt, device="cpu")
        arr = np.frombuffer(blob, dtype=np.uint8)
        return torch.from_numpy(arr.copy() if copy_tensors else arr).view(dt).reshape(shape)

    return _decode(head, make)


# ---- receive buffer pool ---------------------------------------------------------------------------

class ReceiveBufferPool:
    """Bounded, reusable receive storage for ``recv_msg``: the frame is read straight into a pool
    slot and its tensors view that slot, which stays busy until the last such view is gone (freed
    by reference counting, no cyclic GC needed).  A full pool or a failed allocation falls back to
    a frame-owned buffer.  Same limits as the reference's pool (``shard/receive_buffers.py:28-86``):
    budget 1 KiB..512 MiB, 1..64 slots, pinning explicit."""

    def __init__(self, budget_bytes, *, slots=2, pinned=False):
        if type(budget_bytes) is not int or not 1024 <= budget_bytes <= 512 * 1024 ** 2:
            raise ValueError("receive pool budget must be 1KiB..512MiB")
        if type(slots) is not int or not 1 <= slots <= 64 or type(pinned) is not bool:
            raise ValueError("bounded slot count and explicit pinning required")
        if pinned and not torch.cuda.is_available():
            raise RuntimeError("pinned receive pool requires a GPU allocator")
        self.budget_bytes, self.slots, self.pinned = budget_bytes, slots, pinned
        self._lock = threading.Lock()
        self._bufs, self._busy = [], set()
        self.hits = self.fallbacks = self.high_water = self.allocation_failures = 0

    def borrow(self, size):
        """A writable uint8 buffer of `size` bytes tied to a slot, or None (fall back)."""
        if type(size) is not int or size < 0:
            raise ValueError("nonnegative receive frame size required")
        if size == 0:
            return np.empty(0, dtype=np.uint8)
        with self._lock:
            fits = [i for i, b in enumerate(self._bufs) if i not in self._busy and b.numel() >= size]
            if fits:
                index = min(fits, key=lambda i: self._bufs[i].numel())
            else:
                idle = [i for i in range(len(self._bufs)) if i not in self._busy]
                index = min(idle, key=lambda i: self._bufs[i].numel()) if idle else len(self._bufs)
                capacity = max(1024, 1 << max(size - 1, 1).bit_length())
                held = sum(b.numel() for b in self._bufs)   # a resize briefly holds old and new
                if index >= self.slots or held + capacity > self.budget_bytes:
                    self.fallbacks += 1
                    return None
                try:
                    buf = torch.empty(capacity, dtype=torch.uint8, device="cpu", pin_memory=self.pinned)
                except (RuntimeError, OSError, MemoryError):
                    self.fallbacks += 1
                    self.allocation_failures += 1
                    return None
                if index < len(self._bufs):
                    self._bufs[index] = buf
                else:
                    self._bufs.append(buf)
            self._busy.add(index)
            self.hits += 1
            self.high_water = max(self.high_water, len(self._busy))
            # The ctypes array exports the slot's memory; every numpy array / tensor decoded from
            # it keeps it alive, and the slot is released when it is collected.
            exporter = (ctypes.c_uint8 * size).from_address(self._bufs[index].data_ptr())
            weakref.finalize(exporter, self._release, index)
            return np.frombuffer(exporter, dtype=np.uint8)

    def _release(self, index):
        with self._lock:
            self._busy.discard(index)

    def snapshot(self):
        with self._lock:
            held = sum(b.numel() for b in self._bufs)
            return {"schema": "shard-receive-buffer-pool/1", "budget_bytes": self.budget_bytes,
                    "allocated_bytes": held, "slots": self.slots, "live_slots": len(self._busy),
                    "high_water_slots": self.high_water, "borrowed_frames": self.hits,
                    "fallback_frames": self.fallbacks, "allocation_failures": self.allocation_failures,
                    "pinned_allocated_bytes": held if self.pinned else 0, "pinned": self.pinned,
                    "scope": "process lifetime; CPU receive copies only"}


_POOL = None
_POOL_LOCK = threading.Lock()


def configure_receive_pool(budget_bytes=0, *, slots=2, pinned=False):
    """Process-wide opt-in to pooled receive buffers (0 turns it off); refused while a pooled
    frame still has live tensors."""
    global _POOL
    if type(budget_bytes) is not int or budget_bytes < 0 or type(pinned) is not bool:
        raise ValueError("explicit receive buffer budget/pinning required")
    with _POOL_LOCK:
        if _POOL is not None and _POOL.snapshot()["live_slots"]:
            raise RuntimeError("cannot replace a receive pool while tensor views are live")
        _POOL = ReceiveBufferPool(budget_bytes, slots=slots, pinned=pinned) if budget_bytes else None
    return receive_pool_status()


def receive_pool_status():
    pool = _POOL
    return pool.snapshot() if pool is not None else {"enabled": False, "scope": "process lifetime"}


# ---- sockets ---------------------------------------------------------------------------------------

def tune_socket(sock, buf_bytes=SOCK_BUF):
    """Socket buffers large enough for a prefill activation in flight, and no Nagle delay."""
    sock.setsockopt(socket.SOL_SOCKET, socket.SO_SNDBUF, buf_bytes)
    sock.setsockopt(socket.SOL_SOCKET, socket.SO_RCVBUF, buf_bytes)
    if sock.family in (socket.AF_INET, socket.AF_INET6):
        sock.setsockopt(socket.IPPROTO_TCP, socket.TCP_NODELAY, 1)


def _recv_into(sock, view):
    got, n = 0, len(view)
    while got < n:
        r = sock.recv_into(view[got:], n - got)
        if not r:
            try:
                peer = sock.getpeername()
            except (OSError, AttributeError):
                peer = "unknown"
            raise ConnectionError(f"peer {peer} closed the connection while reading a frame ({got}/{n} bytes)")
        got += r


def _recv_exact(sock, n):
    buf = bytearray(n)
    _recv_into(sock, memoryview(buf))
    return buf


def _sendall(sock, parts):
    """sendall of a list of bytes-like segments with scatter/gather sendmsg."""
    bufs = [memoryview(p).cast("B") for p in parts if len(p)]
    if not hasattr(sock, "sendmsg"):
        for b in bufs:
            sock.sendall(b)
        return
    while bufs:
        sent = sock.sendmsg(bufs[:_IOV_MAX])
        while bufs and sent >= len(bufs[0]):
            sent -= len(bufs.pop(0))
        if sent:
            bufs[0] = bufs[0][sent:]


# ---- pinned staging for device tensors -------------------------------------------------------------

class _PinnedRing:
    """RING_SLOTS pinned host chunks and the copy stream their device copies run on, one per device
    and direction.  A transfer holds its ring for its whole frame, so concurrent sends (or
    receives) of one process on one device take turns."""

    def __init__(self, device, chunk_bytes=CHUNK_BYTES, slots=RING_SLOTS):
        self.device = torch.device(device)
        self.chunk = chunk_bytes
        self.bufs = [torch.empty(chunk_bytes, dtype=torch.uint8, pin_memory=True) for _ in range(slots)]
        self.views = [memoryview(b.numpy()) for b in self.bufs]
        self.events = [None] * slots
        self.stream = torch.cuda.Stream(self.device)
        self.lock = threading.Lock()

    def wait_slot(self, s):
        if self.events[s] is not None:
            self.events[s].synchronize()
            self.events[s] = None

    def record(self, s):
        ev = torch.cuda.Event()
        ev.record(self.stream)
        self.events[s] = ev


_RINGS = {}
_RINGS_LOCK = threading.Lock()


def _ring(device, direction):
    key = (torch.device(device).index if torch.device(device).index is not None
           else torch.cuda.current_device(), direction)
    with _RINGS_LOCK:
        if key not in _RINGS:
            _RINGS[key] = _PinnedRing(torch.device("cuda", key[0]))
        return _RINGS[key]


def _send_device_blob(sock, src, ready):
    """Send a device tensor's bytes: chunked D2H into the pinned ring on the copy stream, each
    chunk sent as soon as its copy has landed.  `ready` is an event the copies wait for (the
    producer's stream position)."""
    ring = _ring(src.device, "send")
    k = len(ring.bufs)
    with ring.lock:
        ring.stream.wait_event(ready)
        with torch.cuda.stream(ring.stream):  # a gather of a strided source is ordered after `ready`
            flat = src.contiguous().reshape(-1).view(torch.uint8)
        n = flat.numel()
        n_chunks = (n + ring.chunk - 1) // ring.chunk

        def issue(j):
            s, c0 = j % k, j * ring.chunk
            c1 = min(n, c0 + ring.chunk)
            ring.wait_slot(s)
            with torch.cuda.stream(ring.stream):
                ring.bufs[s][:c1 - c0].copy_(flat[c0:c1], non_blocking=True)
            ring.record(s)

        for j in range(min(k, n_chunks)):
            issue(j)
        for j in range(n_chunks):
            s = j % k
            ring.events[s].synchronize()
            ring.events[s] = None
            _sendall(sock, [ring.views[s][:min(n, (j + 1) * ring.chunk) - j * ring.chunk]])
            if j + k < n_chunks:
                issue(j + k)
        # the source must outlive its copies: every event above has been waited for


def send_msg(sock, obj, ready=None) -> int:
    """Pack and send one message; returns the bytes put on the wire (length prefix included).
    CPU tensors are sent from their own memory; GPU tensors through the pinned ring, after
    `ready` (an event; default: the current stream's position at the call)."""
    head, leaves = _header(obj)
    body = 4 + len(head) + sum(8 + _nbytes(t) for t in leaves)
    segs = [struct.pack("!Q", body), struct.pack("!I", len(head)) + head]
    if any(t.device.type == "cuda" for t in leaves) and ready is None:
        ready = torch.cuda.Event()
        ready.record(torch.cuda.current_stream())
    for t in leaves:
        segs.append(struct.pack("!Q", _nbytes(t)))
        if t.device.type == "cuda":
            if _nbytes(t):
                _sendall(sock, segs)
                segs = []
                _send_device_blob(sock, t, ready)
        else:
            segs.append(_host_bytes(t.cpu()))
    _sendall(sock, segs)
    return 8 + body


def _read_length(sock):
    (n,) = struct.unpack("!Q", _recv_exact(sock, 8))
    if n > MAX_FRAME:
        raise ConnectionError(f"frame length {n} exceeds MAX_FRAME ({MAX_FRAME})")
    return n


_PARSE_ERRORS = (ValueError, KeyError, IndexError, TypeError, RuntimeError, struct.error, json.JSONDecodeError)


def recv_msg(sock):
    """Receive and decode one message into CPU tensors (pool-backed when a receive pool is
    configured).  A frame that does not parse raises ConnectionError (a dead edge)."""
    n = _read_length(sock)
    with _POOL_LOCK:
        pool = _POOL
    frame = pool.borrow(n) if pool is not None else None
    borrowed = frame is not None
    if borrowed:
        _recv_into(sock, memoryview(frame))
    else:
        frame = _recv_exact(sock, n)
    try:
        return _unpack(frame, copy_tensors=not borrowed)
    except _PARSE_ERRORS as e:
        raise ConnectionError(f"malformed frame ({type(e).__name__}: {str(e)[:80]})") from e


def _collect_specs(node, specs):
    """index -> (dtype, shape, nbytes) of every tensor node in a decoded header."""
    if isinstance(node, dict):
        if "__t__" in node:
            dt, shape, nbytes, index = _tensor_spec(node)
            if index in specs and specs[index][2] != nbytes:
                raise ValueError("tensor blob index reused with another size")
            specs[index] = (dt, shape, nbytes)
        else:
            for v in node.values():
                _collect_specs(v, specs)
    elif isinstance(node, list):
        for v in node:
            _collect_specs(v, specs)


def recv_activation(sock, device="cuda"):
    """Receive one message with every tensor placed on `device`: each blob is read chunk by chunk
    into the pinned ring and copied to its device tensor on the copy stream while the next chunk
    arrives.  The current stream is made to wait for the copies before this returns, so the
    tensors are ready for work queued on it.  A malformed frame raises ConnectionError; the
    length, header and every blob size are validated before the device memory is allocated."""
    device = torch.device(device)
    ring = _ring(device, "recv")
    n = _read_length(sock)
    try:
        if n < 4:
            raise ValueError("truncated frame header")
        (hlen,) = struct.unpack("!I", _recv_exact(sock, 4))
        if hlen > n - 4:
            raise ValueError("header length exceeds frame")
        head = json.loads(bytes(_recv_exact(sock, hlen)))
        specs = {}
        _collect_specs(head, specs)
        tensors, left, index, k = {}, n - 4 - hlen, 0, len(ring.bufs)
        with ring.lock:
            while left:
                if left < 8:
                    raise ValueError("truncated blob length")
                (blen,) = struct.unpack("!Q", _recv_exact(sock, 8))
                left -= 8
                if blen > left:
                    raise ValueError("blob length exceeds frame")
                spec = specs.get(index)
                if spec is not None and spec[2] != blen:
                    raise ValueError(f"tensor {spec[1]} needs {spec[2]} bytes, blob has {blen}")
                dst = (torch.empty(blen, dtype=torch.uint8, device=device) if spec is not None else None)
                for j, c0 in enumerate(range(0, blen, ring.chunk)):
                    s, c1 = j % k, min(blen, c0 + ring.chunk)
                    ring.wait_slot(s)
                    _recv_into(sock, ring.views[s][:c1 - c0])
                    if dst is not None:
                        with torch.cuda.stream(ring.stream):
                            dst[c0:c1].copy_(ring.bufs[s][:c1 - c0], non_blocking=True)
                        ring.record(s)
                if dst is not None:
                    dst.record_stream(ring.stream)
                    tensors[index] = dst
                left -= blen
                index += 1
            torch.cuda.current_stream(device).wait_stream(ring.stream)
        if any(i >= index for i in specs):
            raise ValueError("invalid tensor blob index")

        def make(node):
            dt, shape, _, i = _tensor_spec(node)
            if specs[i][2] == 0:
                return torch.empty(shape, dtype=dt, device=device)
            return tensors[i].view(dt).reshape(shape)

        return _decode(head, make)
    except _PARSE_ERRORS as e:
        raise ConnectionError(f"malformed frame ({type(e).__name__}: {str(e)[:80]})") from e


# ---- asynchronous sender ---------------------------------------------------------------------------

def _snapshot(o):
    """The message with every GPU tensor replaced by a copy made on the current stream."""
    if torch.is_tensor(o):
        return o.detach().clone() if o.device.type == "cuda" else o
    if isinstance(o, dict):
        return {k: _snapshot(v) for k, v in o.items()}
    if isinstance(o, (list, tuple)):
        return [_snapshot(v) for v in o]
    return o


class AsyncSender:
    """Sends messages from a background thread in FIFO order, so the stage can compute the next
    chunk while the previous activation drains (the reference's ``_AsyncSender``,
    ``phase0/specpipe.py:313-371``).  ``put`` snapshots GPU tensors on the caller's stream (a
    device-to-device copy) so the caller may overwrite its buffers at once.  A send failure is
    re-raised by the next ``put``; ``close`` is idempotent, discards queued frames and joins with a
    bound."""

    def __init__(self, sock, telemetry=None, maxsize=64):
        self.sock, self.telemetry = sock, telemetry
        self.q = queue.Queue(maxsize=maxsize)
        self.error = None
        self.closed = threading.Event()
        self.thread = threading.Thread(target=self._run, daemon=True)
        self.thread.start()

    def _run(self):
        while not self.closed.is_set():
            try:
                item = self.q.get(timeout=0.25)
            except queue.Empty:
                continue
            if item is None:
                return
            if self.error is not None:
                continue
            obj, ready = item
            try:
                send_msg(self.sock, obj, ready)
            except Exception as e:  # surfaced on the next put()
                self.error = e

    def put(self, obj):
        if self.closed.is_set():
            raise RuntimeError("AsyncSender closed")
        if self.error is not None:
            raise self.error
        ready = None
        obj = _snapshot(obj)
        if torch.cuda.is_available() and torch.cuda.is_initialized():
            ready = torch.cuda.Event()
            ready.record(torch.cuda.current_stream())
        self.q.put((obj, ready))

    def close(self, timeout=5.0):
        self.closed.set()
        try:
            self.sock.shutdown(socket.SHUT_RDWR)
        except (OSError, AttributeError):
            pass
        try:
            self.q.put_nowait(None)
        except queue.Full:
            pass
        self.thread.join(timeout)


# The reference's transport is a drop-in for its PSK wire; with link security handled below the
# engine there is no key to load.
def key_from_env(var: str = "SHARD_PSK") -> None:
    return None


def use_key(material) -> None:
    return None
