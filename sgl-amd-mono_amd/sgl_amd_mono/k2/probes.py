"""Measurement probes behind two design rules of the persistent layer (no counterpart
in the reference): the HBM streaming-read ceiling in the layer's launch shape (one
512-thread workgroup a CU, 16-byte loads, 8 in flight a lane) and a litmus of the
hand-off rules across the eight XCDs' L2 caches.  Both call libmk2.so's
mk2_probe_* entry points on torch's current stream."""

import ctypes

import torch

from .. import _lib

HANDOFF_MODES = {
    0: "write-once, sc1 stores, counter, plain loads",
    1: "write-once, two producers a 128-B line, plain loads",
    2: "line polled (sc1) while partly published, late half read plain",
    3: "line polled (sc1) while partly published, late half read sc1",
}


def _flush(dev, mib=1024):
    # a write larger than the L2s and the 256 MB MALL, so the timed read starts cold
    torch.empty(mib << 20, dtype=torch.uint8, device=dev).fill_(7)


def stream_read(mib, reps=5, launches=20, dev="cuda:0"):
    """Streaming reads of about `mib` MiB a launch (rounded to the probe's unit).
    Returns (bytes, back-to-back GB/s a rep, cold GB/s a rep): back-to-back times
    `launches` launches in a row over distinct buffers cycled through more than 1 GiB
    (so none is still in the L2s or the 256 MB MALL), the way bench.py cycles its
    resident layers; cold times one launch after a 1 GiB flush."""
    lib = _lib.lib()
    unit = lib.mk2_probe_stream_unit()
    if unit == 0:
        raise RuntimeError("mk2_probe_stream_unit: " + lib.mk2_last_error().decode())
    nbytes = max(1, round((mib << 20) / unit)) * unit
    nbuf = max(2, -(-(1 << 30) // nbytes) + 1)
    src = torch.empty(nbuf * nbytes, dtype=torch.uint8, device=dev).fill_(1)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)

    def timed(bufs):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for k in bufs:
            _lib.check(lib.mk2_probe_stream_read(src.data_ptr() + k * nbytes, nbytes, sink.data_ptr(),
                                                 stream.cuda_stream))
        b.record(stream)
        b.synchronize()
        return len(bufs) * nbytes / (a.elapsed_time(b) * 1e-3) / 1e9

    timed([0, 1])  # warm-up
    b2b = [timed([(r * launches + j) % nbuf for j in range(launches)]) for r in range(reps)]
    cold = []
    for _ in range(reps):
        _flush(dev)
        cold.append(timed([0]))
    return nbytes, b2b, cold


def handoff(mode, rounds=100, spin=1 << 18, dev="cuda:0"):
    """One litmus launch; returns (mismatched words, waits that gave up, us a round)."""
    lib = _lib.lib()
    nb, nf = ctypes.c_size_t(), ctypes.c_size_t()
    _lib.check(lib.mk2_probe_handoff_bytes(rounds, ctypes.byref(nb), ctypes.byref(nf)))
    buf = torch.empty(nb.value, dtype=torch.uint8, device=dev)
    flags = torch.empty(nf.value, dtype=torch.uint8, device=dev)
    res = torch.empty(2, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    _lib.check(lib.mk2_probe_handoff(mode, buf.data_ptr(), nb.value, flags.data_ptr(), nf.value, res.data_ptr(),
                                     rounds, spin, stream.cuda_stream))
    b.record(stream)
    b.synchronize()
    r = res.tolist()
    return r[0], r[1], a.elapsed_time(b) * 1e3 / rounds
