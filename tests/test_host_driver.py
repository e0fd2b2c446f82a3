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
                        (["--theta", "0.5"], "--theta"), (["--parts", "3"], "--parts must be"),
                        (["--parts", "4", "--q17"], "excludes --q17")):
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
                                  ["--parts", "4", "--exact"]])
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
