"""Repeatability of the split merge.

A head split across workgroups is finished by whichever split arrives last;
the partials are exchanged through device memory inside one launch.  The
merge reads the partials in split order, so for fixed inputs every launch
must give the same bits whatever the arrival order was.  Each case runs the
same step 2,000 times (the append rewrites the same row with the same bits),
writing every launch's outputs to its own slice, and compares every launch
with the first, in chunks, stopping at the first chunk that differs.
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LAUNCHES = 2000
CHUNK = 250


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("batch,position,split", [(1, 4095, 0), (4, 4095, 256)],
                         ids=["batch1_8splits", "batch4_16splits_of_256"])
def test_split_merge_is_bitwise_repeatable(skv, ctx, batch, position, split):
    _note(f"case: {LAUNCHES} launches, batch {batch}, position {position}, split_tokens {split or 'heuristic'}")
    lut = skv.RopeLut.generate(ctx, 4096)
    kv = skv.KVCache(ctx, layers=1, max_batch=batch, max_seq_len=position + 1)
    kv.fill_synthetic(lut, ntok=position, seed=1234 + batch)
    qkv = [ctx.alloc(batch * 4096 * 4) for _ in range(3)]
    for i, b in enumerate(qkv):
        ctx.fill_synthetic(b, batch * 4096, 1240 + batch, 20 + i)
    row, aq_row, as_row = batch * 4096 * 4, batch * 128 * 56, batch * 128
    outs, aqs, ass = ctx.alloc(CHUNK * row), ctx.alloc(CHUNK * aq_row), ctx.alloc(CHUNK * as_row)
    positions = np.full(batch, position, np.int32)
    ctx.set_split_tokens(split)
    first = None
    try:
        for c0 in range(0, LAUNCHES, CHUNK):
            for i in range(CHUNK):
                skv.swiftkv_attention(ctx, qkv[0], qkv[1], qkv[2], kv, lut, aqs.ptr + i * aq_row,
                                      ass.ptr + i * as_row, 0, positions, outs.ptr + i * row)
            ctx.synchronize()
            o = outs.download(np.uint32, (CHUNK, batch * 4096))
            w = aqs.download(np.uint8, (CHUNK, aq_row))
            e = ass.download(np.uint8, (CHUNK, as_row))
            if first is None:
                first = (o[0].copy(), w[0].copy(), e[0].copy())
                assert np.isfinite(o[0].view(np.float32)).all()
            bad = [c0 + i for i in range(CHUNK)
                   if not (np.array_equal(o[i], first[0]) and np.array_equal(w[i], first[1])
                           and np.array_equal(e[i], first[2]))]
            assert not bad, f"launches {bad[:8]} (of {len(bad)}) differ from launch 0"
            _note(f"  launches {c0 + CHUNK}/{LAUNCHES} identical")
    finally:
        ctx.set_split_tokens(0)
    for b in qkv + [outs, aqs, ass]:
        b.free()
    kv.close()
    lut.close()


@pytest.mark.parametrize("noalloc", [False, True], ids=["context_workspace", "noalloc_workspace"])
def test_split_merge_across_the_tag_wrap(skv, ctx, noalloc):
    """The merge's tags are the (row, head)'s generation + 1, 32 bits, and
    wrap from 0xffffffff to 1 with the head's words cleared.  With every
    generation set just below the wrap, six launches run with tags 0xfffffffd,
    0xfffffffe, 0xffffffff, 1, 2, 3: each must give the bits of a launch far
    from the wrap, on the context's split workspace and on the
    allocation-free entry's."""
    batch, position = 2, 4095     # 4 splits of 1024 tokens per head
    entry = "allocation-free" if noalloc else "regular"
    _note(f"case: tag wrap, batch {batch}, position {position}, {entry} entry")
    lut = skv.RopeLut.generate(ctx, 4096)
    kv = skv.KVCache(ctx, layers=1, max_batch=batch, max_seq_len=position + 1)
    kv.fill_synthetic(lut, ntok=position, seed=77)
    qkv = [ctx.alloc(batch * 4096 * 4) for _ in range(3)]
    for i, b in enumerate(qkv):
        ctx.fill_synthetic(b, batch * 4096, 78, 30 + i)
    out, aq, asc = ctx.alloc(batch * 4096 * 4), ctx.alloc(batch * 128 * 56), ctx.alloc(batch * 128)
    run = skv.swiftkv_attention_noalloc if noalloc else skv.swiftkv_attention
    positions = np.full(batch, position, np.int32)

    def launch():
        run(ctx, qkv[0], qkv[1], qkv[2], kv, lut, aq, asc, 0, positions, out)
        ctx.synchronize()
        return (out.download(np.uint32, (batch * 4096,)), aq.download(np.uint8, (batch * 128 * 56,)),
                asc.download(np.uint8, (batch * 128,)))

    first = launch()
    assert np.isfinite(first[0].view(np.float32)).all()
    ctx.debug_set_split_generation(0xFFFFFFFC, noalloc)
    for i, tag in enumerate([0xFFFFFFFD, 0xFFFFFFFE, 0xFFFFFFFF, 1, 2, 3]):
        got = launch()
        assert all(np.array_equal(g, f) for g, f in zip(got, first)), f"launch {i} (tag {tag:#x}) differs"
        _note(f"  tag {tag:#x}: identical")
    with pytest.raises(skv.SwiftKVError):
        ctx.debug_set_split_generation(0xFFFFFFFF, noalloc)
    for b in qkv + [out, aq, asc]:
        b.free()
    kv.close()
    lut.close()


def test_two_contexts_interleaved(skv, ctx):
    """Two contexts on one GPU, each with its own cache and split workspace,
    their split launches interleaved on two streams: each context's outputs
    equal what it gives alone, bit for bit (every workspace counts its own
    generations, so one context's merges never see the other's words)."""
    _note("case: two contexts, batch 1 (8 splits) and batch 2 (4 splits), interleaved")
    other = skv.Context(0)
    setups = []
    for c, batch, seed in ((ctx, 1, 501), (other, 2, 502)):
        lut = skv.RopeLut.generate(c, 4096)
        kv = skv.KVCache(c, layers=1, max_batch=batch, max_seq_len=4096)
        kv.fill_synthetic(lut, ntok=4095, seed=seed)
        qkv = [c.alloc(batch * 4096 * 4) for _ in range(3)]
        for i, b in enumerate(qkv):
            c.fill_synthetic(b, batch * 4096, seed + 1, 40 + i)
        out = c.alloc(batch * 4096 * 4)
        setups.append((c, batch, lut, kv, qkv, out))

    def launch(s):
        c, batch, lut, kv, qkv, out = s
        skv.swiftkv_attention(c, qkv[0], qkv[1], qkv[2], kv, lut, None, None, 0, np.full(batch, 4095, np.int32), out)

    def result(s):
        s[0].synchronize()
        return s[5].download(np.uint32, (s[1] * 4096,))

    alone = []
    for s in setups:
        launch(s)
        alone.append(result(s))
    for rnd in range(50):
        for s in setups:
            launch(s)
        if rnd % 10 == 9:
            for s, want in zip(setups, alone):
                assert np.array_equal(result(s), want), f"round {rnd}: context with batch {s[1]} differs"
    for c, batch, lut, kv, qkv, out in setups:
        for b in qkv + [out]:
            b.free()
        kv.close()
        lut.close()
    other.close()


@pytest.mark.parametrize("batch,split,noalloc", [(1, 0, False), (4, 256, False), (2, 0, True)],
                         ids=["batch1_8splits_inline_merge", "batch4_16splits_looped_merge", "batch2_noalloc"])
def test_merge_that_gives_up_is_reported(skv, ctx, batch, split, noalloc):
    """A split merge whose wait for another split's partial runs out writes NaN
    into its head's output and must be reported, not pass as success.  The
    testing aid forces it from the host (every merge waits for a tag no
    partial carries and gives up after one poll; every kernel exits
    normally), through the inline merge (up to 8 splits), the looped one (16
    splits) and the allocation-free entry:
      - every merged head's output is NaN and the next synchronize returns
        EHIP naming a cache slot and head, once;
      - a step call issued after a faulting launch has ended returns EHIP and
        enqueues nothing;
      - with the aid off, the next launch gives the bits of a launch before
        the fault: the split workspace stayed consistent."""
    position = 4095
    _note(f"case: merge give-up reported, batch {batch}, split_tokens {split or 'heuristic'}, noalloc={noalloc}")
    lut = skv.RopeLut.generate(ctx, 4096)
    kv = skv.KVCache(ctx, layers=1, max_batch=batch, max_seq_len=position + 1)
    kv.fill_synthetic(lut, ntok=position, seed=990 + batch)
    qkv = [ctx.alloc(batch * 4096 * 4) for _ in range(3)]
    for i, b in enumerate(qkv):
        ctx.fill_synthetic(b, batch * 4096, 991 + batch, 50 + i)
    out, aq, asc = ctx.alloc(batch * 4096 * 4), ctx.alloc(batch * 128 * 56), ctx.alloc(batch * 128)
    run = skv.swiftkv_attention_noalloc if noalloc else skv.swiftkv_attention
    positions = np.full(batch, position, np.int32)

    def enqueue():
        run(ctx, qkv[0], qkv[1], qkv[2], kv, lut, aq, asc, 0, positions, out)

    def result():
        return (out.download(np.uint32, (batch * 4096,)), aq.download(np.uint8, (batch * 128 * 56,)),
                asc.download(np.uint8, (batch * 128,)))

    ctx.set_split_tokens(split)
    try:
        enqueue()
        ctx.synchronize()
        good = result()
        assert np.isfinite(good[0].view(np.float32)).all()
        ctx.debug_force_merge_timeout(True)
        enqueue()
        with pytest.raises(skv.SwiftKVError) as ei:
            ctx.synchronize()
        assert ei.value.code == skv.EHIP and "gave up" in str(ei.value) and "head" in str(ei.value), str(ei.value)
        assert np.isnan(result()[0].view(np.float32)).all()
        ctx.synchronize()                      # reported once
        # a faulting launch that has ended, then a step call: refused, nothing enqueued
        enqueue()
        ctx.timer_record(60)
        ctx.timer_elapsed_ms(60, 60)           # waits for the launch without looking for faults
        sentinel = np.full(batch * 4096, 0x5A5A5A5A, np.uint32)
        out.upload(sentinel)
        with pytest.raises(skv.SwiftKVError) as ei:
            enqueue()
        assert ei.value.code == skv.EHIP
        ctx.synchronize()
        assert np.array_equal(out.download(np.uint32, (batch * 4096,)), sentinel)
        ctx.debug_force_merge_timeout(False)
        enqueue()
        ctx.synchronize()
        again = result()
        assert all(np.array_equal(g, f) for g, f in zip(again, good)), "the launch after the fault differs"
        if not noalloc and split == 0:
            # a recorded graph whose merges give up: its replay is reported, and so
            # is a graph launch after a faulting replay has ended
            ctx.debug_force_merge_timeout(True)
            ctx.capture_begin()
            enqueue()
            g = ctx.capture_end()
            ctx.debug_force_merge_timeout(False)
            g.launch()
            with pytest.raises(skv.SwiftKVError) as ei:
                ctx.synchronize()
            assert ei.value.code == skv.EHIP
            g.launch()
            ctx.timer_record(61)
            ctx.timer_elapsed_ms(61, 61)
            with pytest.raises(skv.SwiftKVError) as ei:
                g.launch()
            assert ei.value.code == skv.EHIP
            ctx.synchronize()
            g.close()
            enqueue()
            ctx.synchronize()
            assert all(np.array_equal(g_, f) for g_, f in zip(result(), good)), "the launch after the graph differs"
    finally:
        ctx.debug_force_merge_timeout(False)
        ctx.set_split_tokens(0)
    for b in qkv + [out, aq, asc]:
        b.free()
    kv.close()
    lut.close()
