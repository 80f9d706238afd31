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
import math
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



def _frame_cap():
    """Largest frame body a receiver accepts, in bytes: M25_MAX_FRAME when set (the reference's knob),
    else 256 MiB.  The length prefix arrives before anything vouches for the sender, so a larger
    claim is refused before a byte of the body is read or allocated."""
    text = os.environ.get("M25_MAX_FRAME", "").strip()
    return int(text) if text else 256 << 20


MAX_FRAME = _frame_cap()
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

_MAX_RANK = 32


class _FrameReader:
    """A cursor over one frame body.  Every length field is checked against the bytes that actually
    follow it before anything is sliced or allocated; a violation raises ValueError, which the
    socket readers turn into a dead-edge ConnectionError."""

    def __init__(self, body):
        self.mv = memoryview(body)
        self.pos = 0

    def left(self):
        return len(self.mv) - self.pos

    def take(self, n, what):
        if n > self.left():
            raise ValueError(f"{what}: {n} bytes declared, {self.left()} remain in the frame")
        out = self.mv[self.pos:self.pos + n]
        self.pos += n
        return out

    def u32(self, what):
        return struct.unpack("!I", self.take(4, what))[0]

    def u64(self, what):
        return struct.unpack("!Q", self.take(8, what))[0]

    def header(self):
        n = self.u32("header length field")
        return json.loads(bytes(self.take(n, "JSON header")))

    def blobs(self):
        out = []
        while self.left():
            n = self.u64(f"length field of blob {len(out)}")
            out.append(self.take(n, f"blob {len(out)}"))
        return out


def _tensor_spec(node, n_blobs=None):
    """Validated (dtype, shape, byte size, blob index) of a header's tensor node."""
    dt = _DTYPES.get(node.get("dtype"))
    if dt is None:
        raise ValueError(f"tensor node with unsupported dtype {node.get('dtype')!r}")
    index = node["__t__"]
    in_range = type(index) is int and index >= 0 and (n_blobs is None or index < n_blobs)
    if not in_range:
        raise ValueError(f"tensor node points at blob {index!r}, frame has {n_blobs}")
    shape = node.get("shape")
    if not (isinstance(shape, list) and len(shape) <= _MAX_RANK and
            all(type(d) is int and d >= 0 for d in shape)):
        raise ValueError(f"tensor shape {shape!r} is not a list of <= {_MAX_RANK} non-negative ints")
    return dt, shape, math.prod(shape) * _ITEMSIZE[dt], index


def _decode(node, make_tensor):
    if isinstance(node, dict):
        if "__t__" in node:
            return make_tensor(node)
        return {k: _decode(v, make_tensor) for k, v in node.items()}
    if isinstance(node, list):
        return [_decode(v, make_tensor) for v in node]
    return node


def _unpack(buf, *, copy_tensors=True):
    """One frame body -> message with CPU tensors.  A tensor's declared shape must account for its
    blob exactly, so no header can make the decoder allocate more than the frame holds.  With
    copy_tensors=False the tensors are views of `buf`, which must outlive them."""
    rd = _FrameReader(buf)
    head = rd.header()
    blobs = rd.blobs()

    def tensor(node):
        dt, shape, nbytes, index = _tensor_spec(node, len(blobs))
        raw = blobs[index]
        if nbytes != len(raw):
            raise ValueError(f"{dt} tensor of shape {shape} is {nbytes} bytes; blob {index} holds {len(raw)}")
        if nbytes == 0:
            return torch.empty(shape, dtype=dt)
        u8 = np.frombuffer(raw, dtype=np.uint8)
        return torch.from_numpy(u8.copy() if copy_tensors else u8).view(dt).reshape(shape)

    return _decode(head, tensor)


# ---- receive buffer pool ---------------------------------------------------------------------------
# Reusable host storage for recv_msg (the reference's opt-in pool, shard/receive_buffers.py:28-86,
# and its process-wide switch, shard/transport.py:64-82).  A frame is read straight into a slot and
# its tensors view the slot, so no second host copy is made.  A slot is leased until the last array
# or tensor viewing it is gone; a full pool, a budget overrun or a failed allocation makes recv_msg
# fall back to a frame-owned buffer.  The status dict follows the "shard-receive-buffer-pool/1" schema
# its callers read (borrowed_frames, live_slots, ...).

_POOL_MIN_BUDGET, _POOL_MAX_BUDGET, _POOL_MAX_SLOTS, _SLOT_MIN = 1 << 10, 512 << 20, 64, 1 << 10


class _Slot:
    __slots__ = ("buf", "leased")

    def __init__(self, buf):
        self.buf, self.leased = buf, False

    @property
    def capacity(self):
        return self.buf.numel()


class ReceiveBufferPool:
    """At most `slots` host buffers (page-locked when `pinned`), each a power of two of at least
    1 KiB, never more than `budget_bytes` in total -- counting, while a slot is regrown, both its old
    and its new buffer."""

    def __init__(self, budget_bytes, *, slots=2, pinned=False):
        if type(budget_bytes) is not int or not _POOL_MIN_BUDGET <= budget_bytes <= _POOL_MAX_BUDGET:
            raise ValueError(f"budget_bytes must be an int in [{_POOL_MIN_BUDGET}, {_POOL_MAX_BUDGET}], "
                             f"got {budget_bytes!r}")
        if type(slots) is not int or not 1 <= slots <= _POOL_MAX_SLOTS:
            raise ValueError(f"slots must be an int in [1, {_POOL_MAX_SLOTS}], got {slots!r}")
        if type(pinned) is not bool:
            raise ValueError(f"pinned must be True or False, got {pinned!r}")
        if pinned and not torch.cuda.is_available():
            raise RuntimeError("page-locked receive slots need the GPU runtime, which is not available")
        self.budget_bytes, self.slots, self.pinned = budget_bytes, slots, pinned
        self._lock = threading.Lock()
        self._table = []                     # _Slot records, at most `slots`
        self.stats = dict(borrowed=0, fallback=0, failed_alloc=0, peak_leased=0)

    def _held(self):
        return sum(sl.capacity for sl in self._table)

    def _find(self, size):
        """An idle slot that already holds `size` bytes (the smallest such), else a slot to (re)grow
        to the next power of two: a new one while the table has room, else the smallest idle one.
        None when neither the table nor the budget allows it."""
        idle = [sl for sl in self._table if not sl.leased]
        fits = [sl for sl in idle if sl.capacity >= size]
        if fits:
            return min(fits, key=lambda sl: sl.capacity)
        want = max(_SLOT_MIN, 1 << (max(size, 2) - 1).bit_length())
        if self._held() + want > self.budget_bytes:
            return None
        try:
            buf = torch.empty(want, dtype=torch.uint8, pin_memory=self.pinned)
        except (RuntimeError, OSError, MemoryError):
            self.stats["failed_alloc"] += 1
            return None
        if len(self._table) < self.slots:
            self._table.append(_Slot(buf))
            return self._table[-1]
        if idle:
            victim = min(idle, key=lambda sl: sl.capacity)
            victim.buf = buf
            return victim
        return None

    def borrow(self, size):
        """A writable uint8 array of exactly `size` bytes leased from a slot, or None."""
        if type(size) is not int or size < 0:
            raise ValueError(f"frame size must be a non-negative int, got {size!r}")
        if size == 0:
            return np.empty(0, dtype=np.uint8)
        with self._lock:
            sl = self._find(size)
            if sl is None:
                self.stats["fallback"] += 1
                return None
            sl.leased = True
            self.stats["borrowed"] += 1
            self.stats["peak_leased"] = max(self.stats["peak_leased"], self.n_leased())
            # a ctypes array owns the lease: every numpy array and tensor decoded from the slot keeps it
            # alive, and collecting it (reference counting alone, no cyclic GC) ends the lease
            owner = (ctypes.c_uint8 * size).from_address(sl.buf.data_ptr())
            weakref.finalize(owner, self._end_lease, sl)
            return np.frombuffer(owner, dtype=np.uint8)

    def _end_lease(self, sl):
        with self._lock:
            sl.leased = False

    def n_leased(self):
        return sum(sl.leased for sl in self._table)

    def snapshot(self):
        with self._lock:
            held = self._held()
            st = self.stats
            return {"schema": "shard-receive-buffer-pool/1", "budget_bytes": self.budget_bytes,
                    "allocated_bytes": held, "slots": self.slots, "live_slots": self.n_leased(),
                    "high_water_slots": st["peak_leased"], "borrowed_frames": st["borrowed"],
                    "fallback_frames": st["fallback"], "allocation_failures": st["failed_alloc"],
                    "pinned_allocated_bytes": held * self.pinned, "pinned": self.pinned,
                    "scope": "per process; host frames of recv_msg"}


_POOL = None
_POOL_LOCK = threading.Lock()


def configure_receive_pool(budget_bytes=0, *, slots=2, pinned=False):
    """Turn pooled receive buffers on for this process (budget_bytes > 0) or off (0).  Refused while
    tensors of a pooled frame are still alive.  Returns the new status."""
    global _POOL
    if type(budget_bytes) is not int or budget_bytes < 0:
        raise ValueError(f"budget_bytes must be a non-negative int, got {budget_bytes!r}")
    if type(pinned) is not bool:
        raise ValueError(f"pinned must be True or False, got {pinned!r}")
    with _POOL_LOCK:
        if _POOL is not None and _POOL.snapshot()["live_slots"]:
            raise RuntimeError("the receive pool still has leased slots: tensor views of pooled frames are live")
        _POOL = ReceiveBufferPool(budget_bytes, slots=slots, pinned=pinned) if budget_bytes else None
    return receive_pool_status()


def receive_pool_status():
    pool = _POOL
    return pool.snapshot() if pool is not None else {"enabled": False, "scope": "per process"}


# ---- sockets ---------------------------------------------------------------------------------------

def tune_socket(sock, buf_bytes=SOCK_BUF):
    """Socket buffers large enough for a prefill activation in flight, and no Nagle delay."""
    sock.setsockopt(socket.SOL_SOCKET, socket.SO_SNDBUF, buf_bytes)
    sock.setsockopt(socket.SOL_SOCKET, socket.SO_RCVBUF, buf_bytes)
    if sock.family in (socket.AF_INET, socket.AF_INET6):
        sock.setsockopt(socket.IPPROTO_TCP, socket.TCP_NODELAY, 1)


def _recv_into(sock, view):
    """Fill `view` from the socket; a peer that hangs up first is a ConnectionError."""
    filled = 0
    while filled < len(view):
        r = sock.recv_into(view[filled:])
        if r == 0:
            raise ConnectionError(f"socket closed by the peer after {filled} of {len(view)} expected bytes")
        filled += r


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
            raise ValueError(f"header length field: 4 bytes declared, {n} remain in the frame")
        (hlen,) = struct.unpack("!I", _recv_exact(sock, 4))
        if hlen > n - 4:
            raise ValueError(f"JSON header: {hlen} bytes declared, {n - 4} remain in the frame")
        head = json.loads(bytes(_recv_exact(sock, hlen)))
        specs = {}
        _collect_specs(head, specs)
        tensors, left, index, k = {}, n - 4 - hlen, 0, len(ring.bufs)
        with ring.lock:
            while left:
                if left < 8:
                    raise ValueError(f"length field of blob {index}: 8 bytes declared, {left} remain in the frame")
                (blen,) = struct.unpack("!Q", _recv_exact(sock, 8))
                left -= 8
                if blen > left:
                    raise ValueError(f"blob {index}: {blen} bytes declared, {left} remain in the frame")
                spec = specs.get(index)
                if spec is not None and spec[2] != blen:
                    raise ValueError(f"{spec[0]} tensor of shape {spec[1]} is {spec[2]} bytes; blob {index} holds {blen}")
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
        missing = [i for i in specs if i >= index]
        if missing:
            raise ValueError(f"tensor node points at blob {missing[0]}, frame has {index}")

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
