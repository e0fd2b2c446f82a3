"""The allocation-free step entry (swiftkv_attention_f32_noalloc) against the
allocating one (swiftkv_attention_f32), through the C ABI.

Two caches are filled identically; each call runs once through each entry on
its own cache, and outputs, A14/E8M0 words and every appended row must be
equal bit for bit.  Two calls in a row: the first a batch of 12 at ragged
positions with forced 512-token splits (up to 8 per head, what the per-GPU
workspace holds), the second smaller -- one sequence with the heuristic's 8
splits -- so the second call runs on what the first left in the shared
workspace.  A call that would split a head more ways than the workspace
holds is refused before any work is enqueued.
"""
import ctypes as C
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _call(skv, fn, ctx, bufs, kv, lut, aq, asc, positions, out):
    pos = np.ascontiguousarray(positions, np.int32)
    return fn(ctx.handle, C.c_void_p(bufs[0].ptr), C.c_void_p(bufs[1].ptr), C.c_void_p(bufs[2].ptr), kv.handle,
              lut.handle, C.c_void_p(aq.ptr), C.c_void_p(asc.ptr), 0, pos.ctypes.data_as(C.c_void_p), pos.size,
              C.c_void_p(out.ptr))


def test_noalloc_entry_matches_the_allocating_entry(skv, ctx):
    L = skv.lib()
    lut = skv.RopeLut.generate(ctx, 4096)
    caches = [skv.KVCache(ctx, layers=1, max_batch=12, max_seq_len=4096) for _ in range(2)]
    for kv in caches:
        kv.fill_synthetic(lut, ntok=4095, seed=515)
    bufs = [ctx.alloc(12 * 4096 * 4) for _ in range(3)]
    for i, b in enumerate(bufs):
        ctx.fill_synthetic(b, 12 * 4096, 516, 40 + i)
    outs = [ctx.alloc(12 * 4096 * 4) for _ in range(2)]
    aqs = [ctx.alloc(12 * 128 * 56) for _ in range(2)]
    ass = [ctx.alloc(12 * 128) for _ in range(2)]
    rng = np.random.default_rng(517)
    calls = [(rng.integers(300, 4096, 12).astype(np.int32), 512), (np.array([4095], np.int32), 0)]
    try:
        for n, (positions, split) in enumerate(calls):
            B = positions.size
            _note(f"case: call {n + 1}, batch {B}, positions up to {positions.max()}, split_tokens {split}")
            ctx.set_split_tokens(split)
            for o in outs:
                o.zero()
            assert _call(skv, L.swiftkv_attention_f32, ctx, bufs, caches[0], lut, aqs[0], ass[0], positions,
                         outs[0]) == skv.OK, L.swiftkv_last_error()
            assert _call(skv, L.swiftkv_attention_f32_noalloc, ctx, bufs, caches[1], lut, aqs[1], ass[1], positions,
                         outs[1]) == skv.OK, L.swiftkv_last_error()
            ctx.synchronize()
            ref, got = (o.download(np.uint32, (B, 4096)) for o in outs)
            assert np.isfinite(ref.view(np.float32)).all()
            assert np.array_equal(ref, got), "FP32 output"
            assert np.array_equal(aqs[0].download(np.uint8, (B, 128, 56)), aqs[1].download(np.uint8, (B, 128, 56)))
            assert np.array_equal(ass[0].download(np.uint8, (B, 128)), ass[1].download(np.uint8, (B, 128)))
            for b in range(B):
                p = int(positions[b])
                for h in (0, 13, 31):
                    x, y = caches[0].read(b, 0, h, p, 1), caches[1].read(b, 0, h, p, 1)
                    assert all(np.array_equal(u, w) for u, w in zip(x, y)), f"appended row, seq {b} head {h}"
        # 256-token splits at position 4095: 16 splits per head, more than the workspace holds; refused
        ctx.set_split_tokens(256)
        before = outs[1].download(np.uint32, (12, 4096))
        rc = _call(skv, L.swiftkv_attention_f32_noalloc, ctx, bufs, caches[1], lut, aqs[1], ass[1],
                   np.array([4095], np.int32), outs[1])
        assert rc == skv.ERANGE and b"allocation-free" in L.swiftkv_last_error()
        ctx.set_split_tokens(0)
        ctx.synchronize()
        assert np.array_equal(outs[1].download(np.uint32, (12, 4096)), before), "a refused call wrote its output"
        # host-memory I/O mode stages through an allocated buffer: refused
        ctx.set_host_io(True)
        try:
            assert _call(skv, L.swiftkv_attention_f32_noalloc, ctx, bufs, caches[1], lut, aqs[1], ass[1],
                         np.array([5], np.int32), outs[1]) == skv.ESTATE
        finally:
            ctx.set_host_io(False)
    finally:
        ctx.set_split_tokens(0)
    for x in bufs + outs + aqs + ass:
        x.free()
    for kv in caches:
        kv.close()
    lut.close()


def test_noalloc_entry_under_graph_capture(skv, ctx):
    """The allocation-free entry recorded into a HIP graph (its purpose: a
    caller under capture cannot allocate): every layer of a 3-sequence step
    at position 2047 (two splits per head, so every head goes through the
    per-GPU workspace), replayed three times with eager calls between the
    replays that advance the workspace's generations (an eager batch-1 call
    with eight splits per head, on the same workspace rows).  Every replay
    must equal the eager step bit for bit."""
    layers, batch, pos = 4, 3, 2047
    _note(f"case: allocation-free entry in a graph, {layers} layers x batch {batch} at position {pos}")
    lut = skv.RopeLut.generate(ctx, 4096)
    kv = skv.KVCache(ctx, layers=layers, max_batch=batch, max_seq_len=2048)
    kv.fill_synthetic(lut, ntok=pos, seed=521)
    n = layers * batch * 4096
    bufs = [ctx.alloc(n * 4) for _ in range(3)]
    for i, b in enumerate(bufs):
        ctx.fill_synthetic(b, n, 522, 60 + i)
    outs = [ctx.alloc(batch * 4096 * 4) for _ in range(layers)]
    aqs = [ctx.alloc(batch * 128 * 56) for _ in range(layers)]
    ass = [ctx.alloc(batch * 128) for _ in range(layers)]
    positions = np.full(batch, pos, np.int32)
    stride = batch * 4096 * 4

    def step():
        for layer in range(layers):
            q, k, v = (b.ptr + layer * stride for b in bufs)
            skv.swiftkv_attention_noalloc(ctx, q, k, v, kv, lut, aqs[layer], ass[layer], layer, positions,
                                          outs[layer])

    def snapshot():
        ctx.synchronize()
        return [(o.download(np.uint32, (batch, 4096)), a.download(np.uint8, (batch, 128, 56)),
                 s.download(np.uint8, (batch, 128))) for o, a, s in zip(outs, aqs, ass)]

    step()
    ref = snapshot()
    for r in ref:
        assert np.isfinite(r[0].view(np.float32)).all()
    extra = ctx.alloc(4096 * 4)
    ctx.capture_begin()
    step()
    g = ctx.capture_end()
    try:
        for rep in range(3):
            for o in outs:
                o.zero()
            ctx.synchronize()
            g.launch()
            got = snapshot()
            for layer in range(layers):
                for x, y in zip(ref[layer], got[layer]):
                    assert np.array_equal(x, y), f"replay {rep}, layer {layer}"
            # eager work between the replays on the same workspace rows
            skv.swiftkv_attention_noalloc(ctx, bufs[0], bufs[1], bufs[2], kv, lut, None, None, 0, [pos], extra)
            ctx.synchronize()
    finally:
        g.close()
    for x in bufs + outs + aqs + ass + [extra]:
        x.free()
    kv.close()
    lut.close()
