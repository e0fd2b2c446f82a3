"""The native host driver (4pe_u250_amd/swiftkv_host, C++ over the C ABI):
argument handling on the CPU, and short runs of every mode on the GPU."""
import json
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST = os.path.join(REPO, "4pe_u250_amd", "swiftkv_host")


def run(*args, timeout=120):
    if not os.path.exists(HOST):
        pytest.fail(f"{HOST} is not built (python 4pe_u250_amd/build.py)")
    return subprocess.run([HOST, *args], capture_output=True, text=True, timeout=timeout)


def test_help_and_argument_errors():
    r = run("--help")
    assert r.returncode == 0 and "--context" in r.stdout and "--rope-lut" in r.stdout
    for bad, needle in ((["--batch", "0"], "--batch 0"), (["--context", "40000"], "--context"),
                        (["--steps", "x"], "--steps x"), (["--frobnicate"], "unknown option"),
                        (["--decode", "--graph"], "cannot advance"), (["--host-io", "--graph"], "cannot be recorded"),
                        (["--context", "32768", "--decode", "--steps", "2"], "beyond the cache limit"),
                        (["--exact", "--context", "4097"], "--exact keeps the reference's bound"),
                        (["--exact", "--context", "4096", "--decode", "--steps", "2"], "positions below 4096"),
                        (["--theta", "0.5"], "--theta"), (["--parts", "3"], "--parts must be"),
                        (["--parts", "4", "--q17"], "excludes --q17"),
                        (["--noalloc", "--q17"], "--noalloc takes FP32 device inputs"),
                        (["--noalloc", "--host-io"], "--noalloc takes FP32 device inputs")):
        r = run(*bad)
        assert r.returncode == 1, bad
        assert needle in r.stderr, (bad, r.stderr)


def test_rope_lut_file_is_size_checked(tmp_path):
    """A file that is not a whole number of 512-byte positions is refused
    before any device work (the checked reader runs after the context, so on
    a machine without a GPU the context error comes first)."""
    bad = tmp_path / "lut.bin"
    bad.write_bytes(b"\0" * 1000)
    r = run("--rope-lut", str(bad), "--context", "1", "--steps", "1", "--layers", "1")
    assert r.returncode == 1
    assert ("holds 1000 bytes" in r.stderr) or ("swiftkv_context_create" in r.stderr), r.stderr


def _result(r):
    assert r.returncode == 0, r.stderr + r.stdout
    line = [ln for ln in r.stdout.splitlines() if ln.startswith("result: ")][-1]
    return json.loads(line[len("result: "):])


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [[], ["--q17"], ["--exact"], ["--graph"], ["--host-io"],
                                  ["--decode", "--t3", "--outliers"], ["--parts", "4"], ["--parts", "2", "--host-io"],
                                  ["--parts", "4", "--exact"], ["--noalloc"], ["--noalloc", "--graph"]])
def test_host_driver_modes(mode):
    print(f"case: swiftkv_host {' '.join(mode)}", flush=True)
    sys.stdout.flush()
    res = _result(run("--layers", "2", "--batch", "3", "--context", "700", "--steps", "3", *mode))
    assert res["us_per_layer"] > 0 and res["gbps"] > 0 and res["max_abs_output"] > 0


@pytest.mark.gpu
def test_host_driver_reference_lut_image(skv, ctx, tmp_path):
    """--rope-lut with an image exported from the library's closed-form table
    (the reference rope_lut.bin's format and values)."""
    lut = skv.RopeLut.generate(ctx, 4096)
    image = tmp_path / "rope_lut.bin"
    image.write_bytes(lut.export(0, 4096))
    lut.close()
    res = _result(run("--rope-lut", str(image), "--layers", "1", "--batch", "2", "--context", "4096",
                      "--steps", "2"))
    assert res["max_abs_output"] > 0


def _dump_inputs(skv, ctx, meta):
    """The driver's q/k/v as the step saw them for the dumped layer: Q15.17
    [batch][4096] each, from the same synthetic streams (FP32, converted as
    the step converts them, or split-K partials reduced and finalized)."""
    import numpy as np
    import oracle as O
    B, L, layer, parts = meta["batch"], meta["layers"], meta["layer"], meta["parts"]
    n_all = L * B * 4096
    out = []
    for i, stream in enumerate(meta["input_streams"]):
        n = parts * n_all
        buf = ctx.alloc(n * 4)
        ctx.fill_synthetic(buf, n, meta["input_seed"], stream, meta["distribution"], meta["outliers"] and i == 1)
        x = buf.download(np.float32, (parts, L, B, 4096))[:, layer]
        buf.free()
        out.append(O.finalize_partials(x) if parts > 1 else O.f2q17(x[0]))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [[], ["--q17"], ["--parts", "4"], ["--exact"], ["--parts", "4", "--exact"],
                                  ["--decode", "--t3", "--outliers"], ["--graph"], ["--host-io"], ["--noalloc"]])
def test_host_driver_dump_matches_the_oracle(skv, ctx, rope_tables, tmp_path, mode):
    """The native host driver's own outputs, dumped with --dump, against the
    oracle on the inputs it generated (the reference host dumps and compares
    its outputs the same way, decode_host.cpp:495-531): the appended row of
    every (sequence, layer, head) bit-exact; the last call's FP32 output
    within tolerance and its A14/E8M0 words bit-exact against the rule, or,
    for --exact, the Q15.17 state and the A14/E8M0 words bit-exact against
    the oracle's integer recurrence."""
    import numpy as np
    import oracle as O
    from gpu_cases import H, assert_close, oracle_cache_synthetic

    print(f"case: swiftkv_host --dump {' '.join(mode)}", flush=True)
    sys.stdout.flush()
    _result(run("--layers", "2", "--batch", "3", "--context", "700", "--steps", "3", "--seed", "91",
                "--dump", str(tmp_path), *mode))
    meta = json.loads((tmp_path / "meta.json").read_text())
    B, L, layer, p0, p = meta["batch"], meta["layers"], meta["layer"], meta["first_position"], meta["position"]
    assert (B, L, layer) == (3, 2, 1) and p == (p0 + 2 if "--decode" in mode else p0) and p0 == 699
    cos, sin = rope_tables
    exact = meta["exact"]
    out = np.fromfile(tmp_path / "output.bin", np.int32 if exact else np.float32).reshape(B, 4096)
    words = np.fromfile(tmp_path / "activation_q.bin", np.uint8).reshape(B, 128, 56)
    codes = np.fromfile(tmp_path / "activation_scale.bin", np.uint8).reshape(B, 128)
    records = np.fromfile(tmp_path / "appended.bin", np.uint8).reshape(B, L, H, 320)

    # every appended row: each layer's own k/v inputs through the append rule at position p
    for lyr in range(L):
        m = dict(meta, layer=lyr)
        _, kq, vq = _dump_inputs(skv, ctx, m)
        for b in range(B):
            krot = O.rope_rotate(kq[b].reshape(H, 128), cos[p], sin[p])
            kc, ks = O.quantize_rows(krot)
            vc, vs = O.quantize_rows(vq[b].reshape(H, 128))
            for h in range(H):
                assert (records[b, lyr, h] == O.pack_record(kc[h], ks[h], vc[h], vs[h])).all(), (b, lyr, h)

    qq, kq, vq = _dump_inputs(skv, ctx, meta)
    for b in range(B):
        sc = oracle_cache_synthetic(skv, ctx, cos, sin, meta["seed"], b, layer, p0, p + 1,
                                    dist=meta["distribution"], k_outliers=meta["outliers"])
        if p > p0:   # --decode: the earlier steps appended the same layer inputs at p0 .. p-1
            sc.fill_q17(np.repeat(kq[b][None], p - p0, 0), np.repeat(vq[b][None], p - p0, 0), p0, cos, sin)
        res = sc.step_q17(qq[b], kq[b], vq[b], p, cos[p], sin[p], fp=not exact, integer=exact)
        if exact:
            assert (out[b] == res["int"].reshape(-1)).all(), f"sequence {b}: Q15.17 state"
            q14, e8 = O.a14_q17(res["int"].reshape(128, 32))
        else:
            assert_close(out[b].reshape(H, 128), res["fp"], f"sequence {b}")
            q14, e8 = O.a14(out[b].reshape(128, 32))
        assert (codes[b] == e8).all() and (words[b] == O.pack_a14(q14)).all(), f"sequence {b}: A14/E8M0"
