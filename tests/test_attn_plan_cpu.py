"""Split plan of the decode attention kernels (csrc/soi_attn_plan.h), built for the host and checked over every
context length.

The plan decides how many workgroups share a KV head's timesteps (the reference's decode_attention,
csrc/kernels/decode_attention.cu:17-63, runs one block per head; the split is this build's). The results do not
depend on it, but the grids do: a device-position launch has cap = min(ceil(L_max / step), ceil(128 / NKV))
splits per KV head, so every length must plan at most that many, and the splits must tile [0, L) exactly.
Checked (3.4 million cases) for L = 1 .. 70000 and a geometric walk to the 2^31 / NKV limit, NKV = 1 .. 64,
step = 16 .. 512:
  * ns = 1 exactly when L fits 8 passes (tps = L then);
  * otherwise tps is a multiple of step and (ns - 1) * tps < L <= ns * tps (no split empty, none missing);
  * ns <= ceil(L / step) and ns <= ceil(128 / NKV) (the grid's cap covers every length);
  * the 32-bit evaluation equals the plan as specified in 64-bit arithmetic: tps = ceil(ceil(L * NKV / G) / step)
    * step with G = 64 up to L * NKV = 8192 rows and 128 above, ns = ceil(L / tps).
"""
import shutil
import subprocess
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parents[1] / "sparse-offload-infer_amd" / "csrc"

HARNESS = r"""
#include <cstdio>
#include "soi_attn_plan.h"
using namespace soi;

static void spec_plan(int64_t L, int64_t NKV, int64_t step, int64_t& tps, int64_t& ns) {
    if (L <= 8 * step) { tps = L; ns = 1; return; }
    const int64_t G = L * NKV <= 8192 ? 64 : 128;
    const int64_t t = ((L * NKV + G - 1) / G + step - 1) / step * step;
    tps = t < step ? step : t;
    ns = (L + tps - 1) / tps;
}

int main() {
    long cases = 0;
    const int64_t nkvs[] = {1, 2, 3, 4, 8, 16, 32, 64};
    for (int64_t step = 16; step <= 512; step *= 2)
        for (int64_t NKV : nkvs) {
            const int64_t limit = (int64_t(1) << 31) / NKV;
            for (int64_t L = 1; L < limit && L <= (int64_t(1) << 30); L = L < 70000 ? L + 1 : L + L / 7 + 1) {
                int tps, ns;
                split_plan(L, NKV, step, tps, ns);
                int64_t st, sn;
                spec_plan(L, NKV, step, st, sn);
                const int64_t cap_len = (L + step - 1) / step, cap_heads = (128 + NKV - 1) / NKV;
                bool ok = tps == st && ns == sn && ns >= 1 && tps >= 1;
                if (L <= 8 * step) ok = ok && ns == 1 && tps == L;
                else ok = ok && tps % step == 0 && int64_t(ns - 1) * tps < L && L <= int64_t(ns) * tps;
                ok = ok && ns <= cap_len && ns <= cap_heads;
                if (!ok) {
                    printf("FAIL L=%lld NKV=%lld step=%lld: tps=%d ns=%d (spec %lld %lld)\n", (long long)L,
                           (long long)NKV, (long long)step, tps, ns, (long long)st, (long long)sn);
                    return 1;
                }
                ++cases;
            }
        }
    printf("%ld cases\n", cases);
    return 0;
}
"""


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    d = tmp_path_factory.mktemp("attn_plan")
    src, exe = d / "plan.cpp", d / "plan"
    src.write_text(HARNESS)
    subprocess.run([gxx, "-O2", "-std=c++17", "-D__host__=", "-D__device__=", "-D__forceinline__=inline",
                    f"-I{CSRC}", "-o", str(exe), str(src)], check=True, capture_output=True, text=True)
    return exe


def test_split_plan_tiles_every_length_within_the_grid_cap(harness):
    r = subprocess.run([str(harness)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert int(r.stdout.split()[0]) > 3_000_000  # every (L, NKV, step) case above
