"""The launchers' grid fold (sw::grid_dim, sw::check_grid in
sparsewavecomp_amd/csrc/sw_internal.h), compiled for the host with g++ and
checked over edge and random sizes: a launch stays 1-D while its x fits
2^32 - 1 work-items; otherwise x * threads stays within that bound, x * y
covers every workgroup, the surplus is less than one workgroup per row
(y - 1 at most, which the kernels' own index checks send home), y fits its
dimension, and check_grid accepts exactly the launches grid_dim can fold.
The kernels number the folded workgroups y * gridDim.x + x (swd::block_id),
so the fold enumerates 0 .. x * y - 1 once each."""
import os
import random
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
UINT32_MAX = 2**32 - 1
MAX_Y = 65535

DRIVER = r'''
#include "sw_internal.h"
#include <cstdio>
int sw::fail(int code, const char *, ...) { return code; }
int main() {
  long long blocks, threads;
  while (std::scanf("%lld %lld", &blocks, &threads) == 2) {
    const dim3 g = sw::grid_dim(blocks, threads);
    std::printf("%u %u %d\n", g.x, g.y,
                sw::check_grid(blocks, threads, "t") == SW_OK);
  }
  return 0;
}
'''


@pytest.fixture(scope="module")
def fold(tmp_path_factory):
    gxx = shutil.which("g++")
    hip = "/opt/rocm/include/hip/hip_runtime.h"
    if gxx is None or not os.path.exists(hip):
        pytest.skip("g++ and the HIP headers are needed")
    d = tmp_path_factory.mktemp("fold")
    src = d / "fold.cpp"
    src.write_text(DRIVER)
    exe = d / "fold"
    subprocess.run([gxx, "-std=c++17", "-D__HIP_PLATFORM_AMD__",
                    "-I/opt/rocm/include",
                    "-I" + os.path.join(ROOT, "sparsewavecomp_amd", "csrc"),
                    str(src), "-o", str(exe)], check=True)

    def run(cases):
        inp = "".join(f"{b} {t}\n" for b, t in cases)
        out = subprocess.run([str(exe)], input=inp, capture_output=True,
                             text=True, check=True).stdout.split("\n")
        return [tuple(int(v) for v in ln.split()) for ln in out if ln]
    return run


def test_fold_properties(fold):
    rng = random.Random(5)
    cases = []
    for threads in (1, 64, 96, 100, 256, 512, 1024):
        row = min(UINT32_MAX // threads, 2**31 - 1)
        for b in (1, 2, row - 1, row, row + 1, 2 * row - 1, 2 * row,
                  2 * row + 1, 3 * row + 7, row * MAX_Y - 1, row * MAX_Y,
                  row * MAX_Y + 1):
            cases.append((b, threads))
        cases += [(rng.randint(1, row * MAX_Y + 10), threads)
                  for _ in range(200)]
    got = fold(cases)
    assert len(got) == len(cases)
    for (blocks, threads), (x, y, ok) in zip(cases, got):
        row = min(UINT32_MAX // threads, 2**31 - 1)
        assert ok == (blocks <= row * MAX_Y), (blocks, threads)
        if not ok:
            continue
        if blocks <= row:
            assert (x, y) == (blocks, 1), (blocks, threads)
            continue
        assert x * threads <= UINT32_MAX, (blocks, threads, x)
        assert 2 <= y <= MAX_Y
        assert x * y >= blocks
        assert x * y - blocks < y, (blocks, threads, x, y)
