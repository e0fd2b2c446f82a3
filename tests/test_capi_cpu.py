"""CPU-only checks of the C ABI: the library loads, exports every symbol that
include/swiftkv.h declares, and rejects bad arguments with the documented
status codes before touching a device.  No compute calls (no GPU here)."""
import ctypes as C
import subprocess

import numpy as np
import pytest


def test_library_exports_every_header_symbol(skv):
    L = skv.lib()
    names = skv.header_symbols()
    assert len(names) >= 30
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(skv._SIGNATURES), "ctypes signature table out of sync with the header"


def test_dynamic_symbol_table(skv):
    out = subprocess.run(["nm", "-D", "--defined-only", skv.LIB_PATH], capture_output=True, text=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    for n in skv.header_symbols():
        assert n in exported, n


def test_built_for_gfx950_only(skv, tmp_path):
    """The offload bundle in .hip_fatbin holds gfx950 code objects only."""
    import re
    blob = tmp_path / "fatbin.bin"
    subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", skv.LIB_PATH, str(blob)], check=True)
    targets = set(re.findall(rb"hipv4-amdgcn-amd-amdhsa--(gfx[0-9a-z]+)", blob.read_bytes()))
    assert targets == {b"gfx950"}


def test_version_and_last_error(skv):
    assert "gfx950" in skv.version()
    assert isinstance(skv.lib().swiftkv_last_error(), bytes)


def test_null_and_range_checks_without_device(skv):
    L = skv.lib()
    assert L.swiftkv_context_create(0, None) == skv.EINVAL
    assert L.swiftkv_synchronize(None) == skv.EINVAL
    assert L.swiftkv_set_split_tokens(None, 256) == skv.EINVAL
    pos = np.array([0], np.int32)
    assert L.swiftkv_attention_f32(None, None, None, None, None, None, None, None, 0,
                                   pos.ctypes.data_as(C.c_void_p), 1, None) == skv.EINVAL
    assert b"null" in L.swiftkv_last_error()
    assert L.swiftkv_rope_lut_export(None, 0, 1, None) == skv.EINVAL
    assert L.swiftkv_kv_cache_bytes(None) == 0
    assert L.swiftkv_rope_lut_positions(None) == 0
    h = C.c_void_p()
    assert L.swiftkv_rope_lut_generate(None, 4096, 10000.0, C.byref(h)) == skv.EINVAL
    assert L.swiftkv_kv_cache_create(None, 1, 1, 1, C.byref(h)) == skv.EINVAL
    assert L.swiftkv_timer_record(None, 0) == skv.EINVAL
    counts = (C.c_int64 * skv.KERNEL_KINDS)()
    ms = (C.c_double * skv.KERNEL_KINDS)()
    assert L.swiftkv_profile_collect(None, counts, ms) == skv.EINVAL
    assert L.swiftkv_set_host_io(None, 1) == skv.EINVAL
    assert L.swiftkv_attention_partials(None, None, None, None, 4, 4096, None, None, None, None, 0,
                                        pos.ctypes.data_as(C.c_void_p), 1, None) == skv.EINVAL
    assert L.swiftkv_convert_partials_q17(None, None, 2, 16, None, 16) == skv.EINVAL
    assert L.swiftkv_attention_exact(None, None, None, None, 0, None, None, None, None, 0,
                                     pos.ctypes.data_as(C.c_void_p), 1, None) == skv.EINVAL
    # destroy functions accept null like free()
    assert L.swiftkv_context_destroy(None) == skv.OK
    assert L.swiftkv_kv_cache_destroy(None) == skv.OK
    assert L.swiftkv_rope_lut_destroy(None) == skv.OK


def test_context_create_reports_the_device_state(skv):
    """The library itself says whether a device is there: with none visible,
    swiftkv_context_create fails with SWIFTKV_EHIP and a HIP message; with one,
    it succeeds for device 0 and refuses an index past the last device with
    SWIFTKV_ERANGE.  Either way no handle is returned on failure."""
    L = skv.lib()
    h = C.c_void_p(1)
    rc = L.swiftkv_context_create(0, C.byref(h))
    if rc == skv.OK:
        assert h.value
        assert L.swiftkv_context_destroy(h) == skv.OK
        h2 = C.c_void_p(1)
        assert L.swiftkv_context_create(4096, C.byref(h2)) == skv.ERANGE
        assert h2.value is None
        assert b"device 4096" in L.swiftkv_last_error()
    else:
        assert rc == skv.EHIP
        assert h.value is None
        assert b"hip" in L.swiftkv_last_error().lower()


def test_unpack_a14_roundtrip(skv, oracle):
    rng = np.random.default_rng(4)
    q = rng.integers(-8191, 8192, (10, 32)).astype(np.int16)
    assert (skv.unpack_a14(oracle.pack_a14(q)) == q).all()


def test_a14_unpack_and_decode_through_the_abi(skv, oracle):
    """The ABI's host unpacker against the oracle's packer (the reference's lane
    layout) and the mirror's independent numpy unpacker; the decode against
    lane * 2^(code - 140) in double precision, saturating to inf like the
    float it returns."""
    rng = np.random.default_rng(5)
    q = rng.integers(-8192, 8192, (300, 32)).astype(np.int16)
    q[0] = 0
    q[1] = -8192
    q[2] = 8191
    q[3, ::2] = -1
    words = oracle.pack_a14(q)
    assert (skv.a14_unpack(words) == q).all()
    assert (skv.unpack_a14(words) == q).all()
    codes = rng.integers(0, 256, 300).astype(np.uint8)
    codes[:4] = [0, 127, 140, 255]
    got = skv.a14_decode(words, codes)
    with np.errstate(over="ignore"):
        want = np.ldexp(q.astype(np.float64), codes.astype(np.int64)[:, None] - 140).astype(np.float32)
    assert (got.view(np.uint32) == want.view(np.uint32)).all()
    L = skv.lib()
    assert L.swiftkv_a14_unpack(None, 1, None) == skv.EINVAL
    assert L.swiftkv_a14_decode(None, None, 1, None) == skv.EINVAL
    assert L.swiftkv_a14_unpack(None, 0, None) == skv.OK


def test_scale_bits(skv, oracle):
    s = np.arange(26, dtype=np.uint8)
    assert (skv.scale_bits(s) == oracle.shift_scale_bits(s)).all()
    assert (skv.scale_bits(s).view(np.float32) == np.ldexp(np.float32(1), s.astype(int) - 17)).all()


def test_host_arrays_need_host_io_mode(skv):
    """A numpy array is host memory: the mirror refuses to hand it to a kernel
    unless the context is in host-memory I/O mode."""
    with pytest.raises(TypeError):
        skv._ptr(np.zeros(4, np.float32))

    class FakeCtx:
        host_io = True
    a = np.zeros(8, np.float32)
    assert skv._io_ptr(FakeCtx, a, np.float32) == a.ctypes.data
    with pytest.raises(TypeError):
        skv._io_ptr(FakeCtx, a, np.int32)
    with pytest.raises(ValueError):
        skv._io_ptr(FakeCtx, np.zeros((4, 4), np.float32)[:, ::2], np.float32)
    with pytest.raises(ValueError):
        skv._check_io_sizes(FakeCtx, 2, np.zeros(4096, np.float32), None, None, None, None, None)


@pytest.mark.parametrize("positions,split,want", [
    ([4095], 0, (512, 8, 8, 32)),              # batch 1: 8 splits, one 8-wave workgroup per CU
    ([2047], 0, (256, 8, 8, 32)),              # batch 1 at context 2048: 256-token splits
    ([4095] * 2, 0, (1024, 4, 8, 32)),
    ([4095] * 4, 0, (2048, 2, 8, 32)),
    ([4095] * 8, 0, (4096, 1, 8, 32)),         # 256 workgroups: no split
    ([4095] * 12, 0, (2048, 2, 8, 32)),        # 768 workgroups: one round of three 4-wave workgroups per CU
    ([4095] * 16, 0, (4096, 1, 8, 32)),
    ([4095] * 24, 0, (4096, 1, 8, 32)),        # 768 workgroups
    ([4095] * 25, 0, (4096, 1, 8, 64)),        # past one round, every range 4096 tokens: 8 waves, 64-token blocks
    ([4095] * 64, 0, (4096, 1, 8, 64)),        # the headline launch
    ([2047] * 32, 0, (2048, 1, 8, 64)),        # ranges of exactly 2048 tokens
    ([2046] * 32, 0, (2048, 1, 4, 64)),        # 2047 tokens: 4 waves
    ([255] + [4095] * 63, 0, (4096, 1, 4, 64)),   # a short row: 4 waves (the ragged batch)
    ([32767] * 16, 0, (8192, 4, 8, 64)),       # no split longer than 8192 tokens
    ([100, 700, 2047], 0, (1024, 2, 8, 32)),
    ([5, 100, 100, 3], 0, (256, 1, 8, 32)),
    ([4095] * 4, 256, (256, 16, 4, 64)),       # forced splits: 2,048 workgroups of 256 tokens
    ([4095], 1536, (1536, 3, 8, 32)),
    ([4095] * 12, 512, (512, 8, 4, 64)),       # 3,072 workgroups
    ([4095] * 32, 2048, (2048, 2, 8, 64)),     # 2,048 workgroups of 2048 tokens
])
def test_step_plan(skv, positions, split, want):
    """The launch plan on the reference device shape (256 CUs, three 4-wave
    step workgroups per CU): tokens per split, splits of the longest
    sequence, waves per workgroup, tokens per block.  Host logic only."""
    got = skv.step_plan(positions, split_tokens=split)
    assert got[:4] == want


def test_step_plan_orders_rows_longest_first(skv):
    split, grid, waves, block, rows = skv.step_plan([5, 100, 100, 3, 4095, 0, 100])
    assert rows.tolist() == [4, 1, 2, 6, 0, 3, 5]       # equal positions keep sequence order
    _, _, _, _, rows = skv.step_plan(list(range(256)))
    assert rows.tolist() == list(range(255, -1, -1))


def test_step_plan_argument_checks(skv):
    L = skv.lib()
    pos = np.array([10, 20], np.int32)
    out = [C.c_int32() for _ in range(3)]
    p = pos.ctypes.data_as(C.c_void_p)

    def plan(cus=256, per_cu=3, split=0, positions=p, batch=2):
        return L.swiftkv_debug_step_plan(cus, per_cu, split, positions, batch, C.byref(out[0]), C.byref(out[1]),
                                         C.byref(out[2]), None, None)

    assert plan() == skv.OK and (out[0].value, out[1].value, out[2].value) == (256, 1, 8)
    assert plan(positions=None) == skv.EINVAL
    assert plan(cus=0) == skv.EINVAL
    assert plan(per_cu=0) == skv.EINVAL
    assert plan(batch=0) == skv.ERANGE
    assert plan(batch=257) == skv.ERANGE
    assert plan(split=300) == skv.EINVAL
    bad = np.array([10, 32768], np.int32)
    assert plan(positions=bad.ctypes.data_as(C.c_void_p)) == skv.ERANGE
    assert b"position 32768" in L.swiftkv_last_error()


def test_bench_reads_committed_profiles():
    """bench.py copies the committed rocprofv3 summaries' figures into its
    roofline; the commit stays text (a hash such as 84e0131 is not a number)."""
    import importlib.util
    import os
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(root, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    for batch, ragged in ((64, False), (1, False), (64, True)):
        vals, path = bench.profile_summary(batch, 4096, ragged)
        assert path is not None, (batch, ragged)
        got = bench.profile_counters(vals)
        assert isinstance(got["commit"], str) and len(got["commit"]) >= 7
        assert 0.99 < got["fetch_ratio"] < 1.1
        assert 0.0 < got["achieved_occupancy_frac"] <= 1.0
        assert got["trace_avg_us"] > 0 and got["bench_ms_per_step"] > 0
    assert bench.profile_summary(3, 4096) == ({}, None)


def test_bench_refuses_more_than_one_gpu():
    """bench.py runs on one GPU: --gpus above 1 exits with a message before any device work."""
    import json
    import os
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in json.loads(r.stdout.strip().splitlines()[-1])["error"]
