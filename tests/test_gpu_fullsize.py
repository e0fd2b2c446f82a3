"""GPU parity at the workload's full sizes.

Caches of these sizes (0.6 GB for 32 layers at batch 1 up to the 77.3 GB
arena of 64 sequences x 32 layers x 4096 tokens) are filled on the device
from synthetic streams through the append rule; the tests regenerate the FP32
source rows of sampled sequences, rebuild them with the oracle and compare:
  - every cached and appended row of the sampled sequences, bit-exact;
  - the appended row of every sequence, bit-exact;
  - the outputs of the sampled sequences within max-abs 2e-5 + rel 1e-4.
"""
import sys

import numpy as np
import pytest

import oracle as O
from gpu_cases import H, assert_close, assert_rows_equal, oracle_cache_synthetic as _oracle_cache

pytestmark = pytest.mark.gpu


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _appended_rows_match(kv, slot, layer, pos, k_f32, v_f32, cos, sin):
    """The row appended at `pos` for every head equals the oracle's append rule."""
    krot = O.rope_rotate(O.f2q17(k_f32).reshape(H, 128), cos[pos], sin[pos])
    kc, ks = O.quantize_rows(krot)
    vc, vs = O.quantize_rows(O.f2q17(v_f32).reshape(H, 128))
    for h in range(H):
        gk, gv, gks, gvs = kv.read(slot, layer, h, pos, 1)
        assert (gk[0] == kc[h]).all() and (gv[0] == vc[h]).all(), f"slot {slot} head {h} position {pos}: codes"
        assert (gks[0].view(np.uint32) == O.shift_scale_bits(ks[h])).all(), f"slot {slot} head {h}: K scales"
        assert (gvs[0].view(np.uint32) == O.shift_scale_bits(vs[h])).all(), f"slot {slot} head {h}: V scales"


def _inputs(skv, ctx, seed, batch, k_outliers=False, dist=0):
    bufs, host = [], []
    for i in range(3):
        b = ctx.alloc(batch * 4096 * 4)
        ctx.fill_synthetic(b, batch * 4096, seed, 9000 + i, dist, k_outliers and i == 1)
        bufs.append(b)
        host.append(b.download(np.float32, (batch, 4096)))
    return bufs, host


def _step(skv, ctx, kv, lut, positions, bufs, out, aq=None, asc=None):
    skv.swiftkv_attention(ctx, bufs[0], bufs[1], bufs[2], kv, lut, aq, asc, 0, positions, out)
    ctx.synchronize()


@pytest.mark.parametrize("ragged", [False, True], ids=["position4095", "ragged256to4095"])
def test_batch64_context4096(skv, ctx, rope_tables, ragged):
    cos, sin = rope_tables
    seed = 4242 + int(ragged)
    rng = np.random.default_rng(seed)
    positions = (rng.integers(255, 4096, 64) if ragged else np.full(64, 4095)).astype(np.int32)
    _note(f"case: batch 64, capacity 4096, {'ragged' if ragged else 'all'} positions, outliers={not ragged}")
    lut = skv.RopeLut.generate(ctx, 4096)
    kv = skv.KVCache(ctx, layers=1, max_batch=64, max_seq_len=4096)
    kv.fill_synthetic(lut, ntok=4095, seed=seed, k_outliers=not ragged)
    bufs, (q, k, v) = _inputs(skv, ctx, seed + 1, 64, k_outliers=not ragged)
    out = ctx.alloc(64 * 4096 * 4)
    aq, asc = ctx.alloc(64 * 128 * 56), ctx.alloc(64 * 128)
    _step(skv, ctx, kv, lut, positions, bufs, out, aq, asc)
    o = out.download(np.float32, (64, H, 128))
    assert np.isfinite(o).all()
    for b in range(64):
        _appended_rows_match(kv, b, 0, int(positions[b]), k[b], v[b], cos, sin)
    sample = sorted({0, 63, int(np.argmin(positions)), int(np.argmax(positions)), 21})
    for b in sample:
        p = int(positions[b])
        _note(f"  oracle check of slot {b}, position {p}")
        sc = _oracle_cache(skv, ctx, cos, sin, seed, b, 0, p, p + 1, k_outliers=not ragged)
        res = sc.step_q17(O.f2q17(q[b]), O.f2q17(k[b]), O.f2q17(v[b]), p, cos[p], sin[p], fp=True)
        assert_rows_equal(kv, sc, b, 0, 0, p + 1)
        assert_close(o[b], res["fp"], f"slot {b} position {p}")
    words = aq.download(np.uint8, (64, 128, 56))
    codes = asc.download(np.uint8, (64, 128))
    for b in (0, 63):
        q14, e8 = O.a14(o[b].reshape(128, 32))
        assert (codes[b] == e8).all() and (words[b] == O.pack_a14(q14)).all()
    for x in bufs + [out, aq, asc]:
        x.free()
    kv.close()
    lut.close()


def _layer_inputs(skv, ctx, seed, layers, batch, k_outliers=False):
    """q/k/v of a whole decode step, [layer][batch][4096] each, on the device
    and on the host."""
    n = layers * batch * 4096
    bufs, host = [], []
    for i in range(3):
        b = ctx.alloc(n * 4)
        ctx.fill_synthetic(b, n, seed, 9100 + i, 0, k_outliers and i == 1)
        bufs.append(b)
        host.append(b.download(np.float32, (layers, batch, 4096)))
    return bufs, host


def _check_sequence_layer(skv, ctx, kv, cos, sin, seed, slot, layer, pos, q, k, v, out_row, aq_row, asc_row,
                          k_outliers=False):
    """Every cached row of (slot, layer) and the appended one bit-exact, the
    output within tolerance, A14/E8M0 bit-exact against the rule."""
    sc = _oracle_cache(skv, ctx, cos, sin, seed, slot, layer, pos, pos + 1, k_outliers=k_outliers)
    res = sc.step_q17(O.f2q17(q), O.f2q17(k), O.f2q17(v), pos, cos[pos], sin[pos], fp=True)
    assert_rows_equal(kv, sc, slot, layer, 0, pos + 1)
    err = assert_close(out_row.reshape(H, 128), res["fp"], f"slot {slot} layer {layer} position {pos}")
    q14, e8 = O.a14(out_row.reshape(128, 32))
    assert (asc_row == e8).all() and (aq_row == O.pack_a14(q14)).all(), f"slot {slot} layer {layer}: A14"
    return err


@pytest.mark.parametrize("position,outliers", [(2047, False), (4095, True)],
                         ids=["position2047", "position4095_outliers"])
def test_batch1_32layer_step(skv, ctx, rope_tables, position, outliers):
    """One full decode step of a 32-layer cache at batch 1: position 2047
    (the 512 MiB cache of 32 x 2048 tokens) and position 4095 with 1% of K
    channels x20.  The 32 per-layer calls run back to back, then layers 0,
    16 and 31 are checked in full against the oracle and every layer's
    appended row bit for bit."""
    cos, sin = rope_tables
    layers, seed = 32, 3100 + position
    _note(f"case: batch 1, 32 layers, position {position}, outliers={outliers}")
    lut = skv.RopeLut.generate(ctx, 4096)
    kv = skv.KVCache(ctx, layers=layers, max_batch=1, max_seq_len=position + 1)
    kv.fill_synthetic(lut, ntok=position, seed=seed, k_outliers=outliers)
    bufs, (q, k, v) = _layer_inputs(skv, ctx, seed + 1, layers, 1, k_outliers=outliers)
    outs = ctx.alloc(layers * 4096 * 4)
    aqs, ass = ctx.alloc(layers * 128 * 56), ctx.alloc(layers * 128)
    for layer in range(layers):
        off = layer * 4096 * 4
        skv.swiftkv_attention(ctx, bufs[0].ptr + off, bufs[1].ptr + off, bufs[2].ptr + off, kv, lut,
                              aqs.ptr + layer * 128 * 56, ass.ptr + layer * 128, layer, [position], outs.ptr + off)
    ctx.synchronize()
    o = outs.download(np.float32, (layers, 4096))
    words = aqs.download(np.uint8, (layers, 128, 56))
    codes = ass.download(np.uint8, (layers, 128))
    assert np.isfinite(o).all()
    for layer in range(layers):
        _appended_rows_match(kv, 0, layer, position, k[layer, 0], v[layer, 0], cos, sin)
    for layer in (0, 16, 31):
        _note(f"  oracle check of layer {layer}")
        _check_sequence_layer(skv, ctx, kv, cos, sin, seed, 0, layer, position, q[layer, 0], k[layer, 0],
                              v[layer, 0], o[layer], words[layer], codes[layer], k_outliers=outliers)
    for x in bufs + [outs, aqs, ass]:
        x.free()
    kv.close()
    lut.close()


@pytest.mark.parametrize("ragged", [False, True], ids=["position4095", "ragged256to4096"])
def test_batch64_32layer_arena(skv, ctx, rope_tables, ragged):
    """The benchmark's arena: 64 sequences x 32 layers x 4096 tokens (77.3 GB),
    filled on the device, one decode step of 32 per-layer calls.  Checked
    against the oracle: (slot 63, layer 31) and (slot 0, layer 0) in full --
    the last and the first page of the arena -- plus the longest and the
    shortest sequence on layer 17, and every slot's appended row on layers 0
    and 31.  The ragged case draws attended lengths from U{256..4096}."""
    cos, sin = rope_tables
    layers, batch, seed = 32, 64, 6400 + int(ragged)
    rng = np.random.default_rng(seed)
    positions = (rng.integers(256, 4097, batch) - 1 if ragged else np.full(batch, 4095)).astype(np.int32)
    _note(f"case: batch 64 x 32 layers x capacity 4096 arena, {'ragged' if ragged else 'uniform'} positions")
    lut = skv.RopeLut.generate(ctx, 4096)
    kv = skv.KVCache(ctx, layers=layers, max_batch=batch, max_seq_len=4096)
    assert kv.nbytes == 64 * 32 * 32 * 4096 * 288
    kv.fill_synthetic(lut, ntok=4095, seed=seed)
    bufs, (q, k, v) = _layer_inputs(skv, ctx, seed + 1, layers, batch)
    outs = ctx.alloc(layers * batch * 4096 * 4)
    aqs, ass = ctx.alloc(layers * batch * 128 * 56), ctx.alloc(layers * batch * 128)
    stride = batch * 4096 * 4
    for layer in range(layers):
        skv.swiftkv_attention(ctx, bufs[0].ptr + layer * stride, bufs[1].ptr + layer * stride,
                              bufs[2].ptr + layer * stride, kv, lut, aqs.ptr + layer * batch * 128 * 56,
                              ass.ptr + layer * batch * 128, layer, positions, outs.ptr + layer * stride)
    ctx.synchronize()
    _note("  step done")
    o = outs.download(np.float32, (layers, batch, 4096))
    assert np.isfinite(o).all()
    for layer in (0, 31):
        for b in range(batch):
            _appended_rows_match(kv, b, layer, int(positions[b]), k[layer, b], v[layer, b], cos, sin)
    checks = [(63, 31), (0, 0), (int(np.argmax(positions)), 17), (int(np.argmin(positions)), 17)]
    for slot, layer in checks:
        p = int(positions[slot])
        _note(f"  oracle check of slot {slot}, layer {layer}, position {p}")
        words = aqs.download(np.uint8, (128, 56), offset=(layer * batch + slot) * 128 * 56)
        codes = ass.download(np.uint8, (128,), offset=(layer * batch + slot) * 128)
        _check_sequence_layer(skv, ctx, kv, cos, sin, seed, slot, layer, p, q[layer, slot], k[layer, slot],
                              v[layer, slot], o[layer, slot], words, codes)
    for x in bufs + [outs, aqs, ass]:
        x.free()
    kv.close()
    lut.close()


@pytest.mark.parametrize("entry", ["regular", "noalloc"])
@pytest.mark.parametrize("kind", ["ragged", "uniform"])
def test_batch300_split_across_two_launches(skv, ctx, rope_tables, entry, kind):
    """300 sequences at ragged positions 300..1400 (or all at position 1400)
    with forced 256-token splits: two launches (256 rows, then 44) whose split
    heads reuse the same workspace rows (the second launch's tags follow the
    first's), through the regular entry and through the allocation-free one,
    whose fixed workspace holds the split slots of 32 sequences, so it runs
    them as 10 launches of at most 32 sequences with the same plan: its
    outputs must equal the regular entry's bit for bit.  A launch whose
    sequences share one position computes its rows in the kernel instead of
    reading them (the uniform case, whose launches start at cache slots 0,
    32, ..., 256).  Every sequence's appended row bit-exact; the outputs of
    sequences on both sides of the launch boundaries checked in full against
    the oracle."""
    cos, sin = rope_tables
    batch, seed = 300, 7300
    rng = np.random.default_rng(seed)
    positions = rng.integers(300, 1401, batch).astype(np.int32)
    if kind == "uniform":
        positions[:] = 1400
    _note(f"case: batch {batch}, {kind} positions up to 1400, 256-token splits, {entry} entry")
    lut = skv.RopeLut.generate(ctx, 4096)
    kv = skv.KVCache(ctx, layers=1, max_batch=batch, max_seq_len=1408)
    kv.fill_synthetic(lut, ntok=1400, seed=seed)
    n = batch * 4096
    bufs, host = [], []
    for i in range(3):
        b = ctx.alloc(n * 4)
        ctx.fill_synthetic(b, n, seed + 1, 9200 + i)
        bufs.append(b)
        host.append(b.download(np.float32, (batch, 4096)))
    q, k, v = host
    out, aq, asc = ctx.alloc(n * 4), ctx.alloc(batch * 128 * 56), ctx.alloc(batch * 128)
    run = skv.swiftkv_attention_noalloc if entry == "noalloc" else skv.swiftkv_attention
    ctx.set_split_tokens(256)
    try:
        for _ in range(2):   # twice: the second call's tags follow the first's
            run(ctx, bufs[0], bufs[1], bufs[2], kv, lut, aq, asc, 0, positions, out)
        ctx.synchronize()
    finally:
        ctx.set_split_tokens(0)
    o = out.download(np.float32, (batch, 4096))
    words = aq.download(np.uint8, (batch, 128, 56))
    codes = asc.download(np.uint8, (batch, 128))
    assert np.isfinite(o).all()
    if entry == "noalloc":
        ctx.set_split_tokens(256)
        try:
            skv.swiftkv_attention(ctx, bufs[0], bufs[1], bufs[2], kv, lut, aq, asc, 0, positions, out)
            ctx.synchronize()
        finally:
            ctx.set_split_tokens(0)
        assert np.array_equal(out.download(np.float32, (batch, 4096)).view(np.uint32), o.view(np.uint32))
        assert np.array_equal(aq.download(np.uint8, (batch, 128, 56)), words)
        assert np.array_equal(asc.download(np.uint8, (batch, 128)), codes)
    for b in range(batch):
        _appended_rows_match(kv, b, 0, int(positions[b]), k[b], v[b], cos, sin)
    for b in (0, 31, 32, 255, 256, 299, int(np.argmax(positions))):
        p = int(positions[b])
        _note(f"  oracle check of sequence {b}, position {p}")
        sc = _oracle_cache(skv, ctx, cos, sin, seed, b, 0, p, p + 1)
        res = sc.step_q17(O.f2q17(q[b]), O.f2q17(k[b]), O.f2q17(v[b]), p, cos[p], sin[p], fp=True)
        assert_rows_equal(kv, sc, b, 0, 0, p + 1)
        assert_close(o[b].reshape(H, 128), res["fp"], f"sequence {b} position {p}")
        q14, e8 = O.a14(o[b].reshape(128, 32))
        assert (codes[b] == e8).all() and (words[b] == O.pack_a14(q14)).all(), f"sequence {b}: A14"
    for x in bufs + [out, aq, asc]:
        x.free()
    kv.close()
    lut.close()


def test_batch16_context32k_512_steps(skv, ctx):
    """Config-5 shape: 16 sequences, unit-variance Student-t(3) rows, cache
    pre-filled to 32256 tokens, then 512 consecutive decode steps to 32767
    (beyond the reference's 4096 limit: RoPE table extended by its closed
    form, FP32 formula as the oracle)."""
    B, start, steps, cap = 16, 32256, 512, 32768
    seed = 5150
    _note(f"case: batch {B}, context {start}..{start + steps}, Student-t(3), {steps} steps")
    cos, sin = O.rope_values(cap)
    lut = skv.RopeLut.generate(ctx, cap)
    kv = skv.KVCache(ctx, layers=1, max_batch=B, max_seq_len=cap)
    kv.fill_synthetic(lut, ntok=start, seed=seed, dist=skv.DIST_STUDENT_T3)
    n = steps * B * 4096
    qkv = [ctx.alloc(n * 4) for _ in range(3)]
    for i, b in enumerate(qkv):
        ctx.fill_synthetic(b, n, seed + 1, 7000 + i, skv.DIST_STUDENT_T3)
    outs = ctx.alloc(steps * B * 4096 * 4)
    stride = B * 4096 * 4
    for j in range(steps):
        off = j * stride
        skv.swiftkv_attention(ctx, qkv[0].ptr + off, qkv[1].ptr + off, qkv[2].ptr + off, kv, lut, None, None, 0,
                              np.full(B, start + j, np.int32), outs.ptr + off)
        if j % 128 == 127:
            ctx.synchronize()
            _note(f"  step {j + 1}/{steps}")
    ctx.synchronize()
    q, k, v = (b.download(np.float32, (steps, B, 4096)) for b in qkv)
    o = outs.download(np.float32, (steps, B, H, 128))
    assert np.isfinite(o).all()
    # every appended row of every sequence
    _note("  checking appended rows")
    for b in range(B):
        for h in range(H):
            gk, gv, gks, gvs = kv.read(b, 0, h, start, steps)
            krot = O.rope_rotate(O.f2q17(k[:, b, h * 128:(h + 1) * 128]), cos[start:start + steps],
                                 sin[start:start + steps])
            kc, ks = O.quantize_rows(krot)
            vc, vs = O.quantize_rows(O.f2q17(v[:, b, h * 128:(h + 1) * 128]))
            assert (gk == kc).all() and (gv == vc).all(), f"slot {b} head {h}: appended codes"
            assert (gks.view(np.uint32) == O.shift_scale_bits(ks)).all()
            assert (gvs.view(np.uint32) == O.shift_scale_bits(vs)).all()
    # outputs of the first and the last step for one sequence
    _note("  oracle check of slot 5")
    b = 5
    sc = _oracle_cache(skv, ctx, cos, sin, seed, b, 0, start, cap, dist=skv.DIST_STUDENT_T3)
    res = sc.step_q17(O.f2q17(q[0, b]), O.f2q17(k[0, b]), O.f2q17(v[0, b]), start, cos[start], sin[start])
    assert_close(o[0, b], res["fp"], "first step")
    sc.fill_q17(O.f2q17(k[1:steps - 1, b]), O.f2q17(v[1:steps - 1, b]), start + 1, cos, sin)
    last = start + steps - 1
    res = sc.step_q17(O.f2q17(q[-1, b]), O.f2q17(k[-1, b]), O.f2q17(v[-1, b]), last, cos[last], sin[last])
    assert_close(o[-1, b], res["fp"], "last step")
    assert_rows_equal(kv, sc, b, 0, 0, last + 1, heads=(0, 9, 31))
    for x in qkv + [outs]:
        x.free()
    kv.close()
    lut.close()
