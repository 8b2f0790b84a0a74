"""sin^2 of the speech decoder's SnakeBeta epilogues (csrc/qtts_snake.h),
compiled for the host with g++ and checked against float64 sin^2.

The reference squares a correctly rounded f32 sin (snake_beta,
conv.rs:620-640).  Bar: over |t| < 2^14 the absolute error stays within
1.3e-7, the largest error of squaring a correctly rounded sin in f32 on
the same arguments; beyond it (the sinf branch), inf and NaN behave as
sinf does.  A sign or coefficient slip, a dropped series term or a swapped
quadrant parity each exceed the bar by a factor of two or more.
"""
import os
import shutil
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "qora-tts-12hz-1.7b_amd", "csrc")

DRIVER = r"""
#include "qtts_snake.h"
#include <cstdio>
#include <vector>
int main(int argc, char **argv)
{
    FILE *f = fopen(argv[1], "rb");
    std::vector<float> t;
    float v;
    while (fread(&v, 4, 1, f) == 1) t.push_back(v);
    fclose(f);
    FILE *g = fopen(argv[2], "wb");
    for (float x : t) {
        const float y = qtts::snake_sin2(x);
        fwrite(&y, 4, 1, g);
    }
    fclose(g);
    return 0;
}
"""


@pytest.fixture(scope="module")
def sin2(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    d = tmp_path_factory.mktemp("snake")
    src, exe = d / "drv.cpp", d / "drv"
    src.write_text(DRIVER)
    subprocess.run(["g++", "-std=c++17", "-O2", "-ffp-contract=off", "-I", CSRC, str(src), "-o", str(exe)],
                   check=True)

    def run(t):
        t = np.ascontiguousarray(t, np.float32)
        (d / "in.bin").write_bytes(t.tobytes())
        subprocess.run([str(exe), str(d / "in.bin"), str(d / "out.bin")], check=True)
        return np.frombuffer((d / "out.bin").read_bytes(), np.float32)

    return run


def arguments(rng):
    parts = [rng.uniform(-lim, lim, 400_000) for lim in (1.0, 10.0, 100.0, 1000.0, 16383.0)]
    parts.append(10.0 ** rng.uniform(-30, 0, 100_000) * rng.choice([-1.0, 1.0], 100_000))
    k = rng.integers(-10_000, 10_000, 200_000)   # next to multiples of pi/2, where sin^2 or cos^2 -> 0
    parts.append(k * (np.pi / 2) + rng.uniform(-1e-3, 1e-3, k.size))
    return np.concatenate(parts).astype(np.float32)


def test_sin2_error_within_a_rounded_sin_squared(sin2):
    t = arguments(np.random.default_rng(7))
    got = sin2(t).astype(np.float64)
    truth = np.sin(t.astype(np.float64)) ** 2
    err = np.abs(got - truth)
    assert err.max() <= 1.3e-7, f"max abs err {err.max():.3e} at t={t[err.argmax()]!r}"
    # and within the ulp envelope of the product: a handful of ulp of sin^2
    ulp = np.spacing(np.maximum(truth, 1e-38).astype(np.float32)).astype(np.float64)
    assert (err / ulp).max() <= 4.0


def test_sin2_special_values(sin2):
    t = np.array([0.0, -0.0, np.pi / 2, -np.pi / 2, np.pi, 16384.0, -16384.0, 1e6, 3e38,
                  np.inf, -np.inf, np.nan], np.float32)
    got = sin2(t)
    assert got[0] == 0.0 and got[1] == 0.0
    assert abs(got[2] - 1.0) <= 1.2e-7 and abs(got[3] - 1.0) <= 1.2e-7
    assert abs(got[4]) <= 1e-13
    big = np.sin(t[5:9].astype(np.float64)) ** 2   # the sinf branch
    assert np.all(np.abs(got[5:9] - big) <= 2.5e-7)
    assert np.all(np.isnan(got[9:]))


def test_sin2_matches_tiny_argument_limit(sin2):
    # t -> 0: sin^2 t = t^2 (1 - t^2/3 + ...), relative error a few ulp
    t = (10.0 ** np.linspace(-19, -2, 2000)).astype(np.float32)
    got = sin2(t).astype(np.float64)
    truth = np.sin(t.astype(np.float64)) ** 2
    assert np.all(np.abs(got - truth) <= 4 * np.spacing(truth.astype(np.float32)).astype(np.float64))
