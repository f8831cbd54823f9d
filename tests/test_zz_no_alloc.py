"""GPU: the allocation-free sampler entry point (mg_sample_logits_noalloc).

It must give exactly what mg_sample_logits gives for the same logits and
generator states (tokens and advanced states), on device buffers the caller
owns, with its scratch counters cleared between calls: two calls in a row, the
second with fewer rows, then a greedy call, a non-finite row and the row limit;
and captured into a HIP graph, replayed with new inputs between replays.
"""
import ctypes

import numpy as np
import pytest

import grokking_abmod_amd as G

pytestmark = pytest.mark.gpu


class DeviceBuffers:
    """hipMalloc'd buffers for the caller's side of the entry point."""

    def __init__(self):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        self.hip.hipFree.argtypes = [ctypes.c_void_p]
        self.hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        self.hip.hipDeviceSynchronize.argtypes = []
        self.ptrs = []

    def alloc(self, nbytes):
        p = ctypes.c_void_p()
        assert self.hip.hipMalloc(ctypes.byref(p), max(int(nbytes), 16)) == 0
        self.ptrs.append(p.value)
        return p.value

    def upload(self, array):
        array = np.ascontiguousarray(array)
        p = self.alloc(array.nbytes)
        assert self.hip.hipMemcpy(p, array.ctypes.data, array.nbytes, 1) == 0
        return p

    def download(self, p, shape, dtype):
        out = np.empty(shape, dtype=dtype)
        assert self.hip.hipDeviceSynchronize() == 0
        assert self.hip.hipMemcpy(out.ctypes.data, p, out.nbytes, 2) == 0
        return out

    def free(self):
        for p in self.ptrs:
            self.hip.hipFree(p)
        self.ptrs = []


def run_noalloc(buf, logits, temperature, states):
    rows, vocab = logits.shape
    d_logits = buf.upload(logits.astype(np.float32))
    d_states = buf.upload(np.asarray(states, dtype=np.uint64))
    d_tokens = buf.upload(np.full(rows, 0xFFFFFFFF, dtype=np.uint32))
    d_flag = buf.upload(np.array([7], dtype=np.int32))
    G.sample_logits_noalloc(d_logits, rows, vocab, temperature, d_states, d_tokens, d_flag)
    return (buf.download(d_tokens, rows, np.uint32), buf.download(d_states, rows, np.uint64),
            int(buf.download(d_flag, 1, np.int32)[0]))


def test_noalloc_sampler_matches_the_allocating_entry_point():
    rng = np.random.default_rng(2024)
    buf = DeviceBuffers()
    try:
        for k, (rows, vocab, T) in enumerate([(300, 256, 0.8), (37, 1000, 1.3)]):
            logits = (rng.normal(size=(rows, vocab)) * 2).astype(np.float32)
            states = rng.integers(0, 2**63, rows, dtype=np.uint64)
            want_tokens, want_states = G.sample_logits(logits, T, states)
            tokens, new_states, flag = run_noalloc(buf, logits, T, states)
            assert np.array_equal(tokens, want_tokens), f"call {k}"
            assert np.array_equal(new_states, want_states), f"call {k}"
            assert flag == 0
        # Greedy: the first maximal logit, states untouched.
        logits = (rng.normal(size=(64, 256))).astype(np.float32)
        logits[3, 10] = logits[3, 20] = logits[3].max() + 1.0
        states = rng.integers(0, 2**63, 64, dtype=np.uint64)
        tokens, new_states, flag = run_noalloc(buf, logits, 0.0, states)
        assert np.array_equal(tokens, np.argmax(logits, axis=1)) and tokens[3] == 10
        assert np.array_equal(new_states, states) and flag == 0
        # A non-finite row sets the flag; the finite rows draw as before.
        logits = (rng.normal(size=(16, 256))).astype(np.float32)
        logits[5, 7] = np.nan
        states = rng.integers(0, 2**63, 16, dtype=np.uint64)
        tokens, _, flag = run_noalloc(buf, logits, 0.9, states)
        assert flag == 1
        finite = np.arange(16) != 5
        want_tokens, _ = G.sample_logits(logits[finite], 0.9, states[finite])
        assert np.array_equal(tokens[finite], want_tokens)
    finally:
        buf.free()


def test_noalloc_sampler_replays_under_graph_capture():
    """The stated use: the call captured into a HIP graph (global capture mode,
    the strictest), the graph replayed three times with eager work between the
    replays (new logits, reset outputs), each replay checked against
    mg_sample_logits on the states the previous one left; the caller's current
    device is unchanged by the call."""
    hip = ctypes.CDLL("libamdhip64.so")
    vp = ctypes.c_void_p
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(vp)]
    hip.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
    hip.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
    hip.hipGraphInstantiate.argtypes = [ctypes.POINTER(vp), vp, vp, vp, ctypes.c_size_t]
    hip.hipGraphLaunch.argtypes = [vp, vp]
    hip.hipStreamSynchronize.argtypes = [vp]
    hip.hipGraphExecDestroy.argtypes = [vp]
    hip.hipGraphDestroy.argtypes = [vp]
    hip.hipStreamDestroy.argtypes = [vp]
    hip.hipGetDevice.argtypes = [ctypes.POINTER(ctypes.c_int)]
    rng = np.random.default_rng(77)
    rows, vocab, T = 96, 256, 0.9
    buf = DeviceBuffers()
    stream, graph, exe = vp(), vp(), vp()
    try:
        logits = (rng.normal(size=(rows, vocab)) * 2).astype(np.float32)
        states = rng.integers(0, 2**63, rows, dtype=np.uint64)
        d_logits = buf.upload(logits)
        d_states = buf.upload(states)
        d_tokens = buf.upload(np.full(rows, 0xFFFFFFFF, dtype=np.uint32))
        d_flag = buf.upload(np.array([7], dtype=np.int32))
        assert hip.hipStreamCreate(ctypes.byref(stream)) == 0
        before = ctypes.c_int(-1)
        assert hip.hipGetDevice(ctypes.byref(before)) == 0
        # An eager call first: the scratch address is looked up outside capture.
        G.sample_logits_noalloc(d_logits, rows, vocab, T, d_states, d_tokens, d_flag, stream=stream.value)
        assert hip.hipStreamSynchronize(stream) == 0
        want_tokens, states = G.sample_logits(logits, T, states)
        assert np.array_equal(buf.download(d_tokens, rows, np.uint32), want_tokens)
        assert np.array_equal(buf.download(d_states, rows, np.uint64), states)
        assert hip.hipStreamBeginCapture(stream, 0) == 0  # hipStreamCaptureModeGlobal
        G.sample_logits_noalloc(d_logits, rows, vocab, T, d_states, d_tokens, d_flag, stream=stream.value)
        assert hip.hipStreamEndCapture(stream, ctypes.byref(graph)) == 0
        after = ctypes.c_int(-1)
        assert hip.hipGetDevice(ctypes.byref(after)) == 0 and after.value == before.value
        assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        for replay in range(3):
            if replay == 2:
                logits[7, 3] = np.inf  # a non-finite row in the last replay
            else:
                logits = (rng.normal(size=(rows, vocab)) * (1 + replay)).astype(np.float32)
            assert buf.hip.hipMemcpy(d_logits, logits.ctypes.data, logits.nbytes, 1) == 0
            sentinel = np.full(rows, 0xFFFFFFFF, dtype=np.uint32)
            assert buf.hip.hipMemcpy(d_tokens, sentinel.ctypes.data, sentinel.nbytes, 1) == 0
            flag = np.array([7], dtype=np.int32)
            assert buf.hip.hipMemcpy(d_flag, flag.ctypes.data, 4, 1) == 0
            assert hip.hipGraphLaunch(exe, stream) == 0
            assert hip.hipStreamSynchronize(stream) == 0
            tokens = buf.download(d_tokens, rows, np.uint32)
            got_states = buf.download(d_states, rows, np.uint64)
            got_flag = int(buf.download(d_flag, 1, np.int32)[0])
            finite = np.isfinite(logits).all(axis=1)
            want_tokens, want_states = G.sample_logits(logits[finite], T, states[finite])
            assert np.array_equal(tokens[finite], want_tokens), f"replay {replay}"
            assert np.array_equal(got_states[finite], want_states), f"replay {replay}"
            assert got_flag == (0 if finite.all() else 1), f"replay {replay}"
            states = got_states
    finally:
        if exe.value:
            hip.hipGraphExecDestroy(exe)
        if graph.value:
            hip.hipGraphDestroy(graph)
        if stream.value:
            hip.hipStreamDestroy(stream)
        buf.free()


def test_noalloc_sampler_rejects_rows_beyond_its_scratch():
    with pytest.raises(G.MeshGptError, match="at most 65536 rows"):
        G.sample_logits_noalloc(16, 65537, 256, 1.0, 16, 16, 16)
