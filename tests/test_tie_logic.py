"""The closed-form 2-of-4 keep logic of the device code (sf_common.hpp: topk2_keep_rel,
topk2_spread_f / topk2_keep_f, the "spread" form used for flip counting) against torch.topk's
tie order, on the host.

Both functions are __host__ __device__, so a small host program built with hipcc evaluates
them on every pattern of the fixture tests/golden/topk_ties_m4.json (all 75 weak orderings
of four values, written from torch.topk) and on a 7-level grid of all 2401 4-tuples with
-0.0 / +0.0 ties; the expected keep sets come from the fixture's k = 2 table.
"""
import json
import os
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(REPO, "tests", "golden")

HARNESS = r"""
#include "sf_common.hpp"
#include <cstdio>
namespace sf { void set_error(const char*, ...) {} }
int main() {
  float v[4];
  while (scanf("%f %f %f %f", &v[0], &v[1], &v[2], &v[3]) == 4) {
    const uint32_t rel = sf::topk2_keep_rel(v[1] >= v[0], v[2] >= v[0], v[3] >= v[0], v[2] >= v[1], v[3] >= v[1],
                                            v[3] >= v[2], v[1] == v[2], v[1] == v[3], v[2] == v[3]);
    const uint32_t spread = sf::topk2_spread_f(v);
    printf("%u %u %u\n", rel, sf::topk2_keep_f(v), spread);
  }
  return 0;
}
"""


def _torch_keep(vals, table):
    """Keep set of torch.topk(2) for vals, through the fixture: rank key sum_i lt_i << 2i."""
    key = 0
    for i, x in enumerate(vals):
        key |= sum(1 for y in vals if y < x) << (2 * i)
    return table[str(key)]["keep"]


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    d = tmp_path_factory.mktemp("ties")
    src, exe = d / "ties.cpp", d / "ties"
    src.write_text(HARNESS)
    subprocess.run([hipcc, "-x", "hip", "--offload-arch=gfx950", "-O1", "-I",
                    os.path.join(REPO, "sparseforge_amd", "csrc"), "-o", str(exe), str(src)],
                   check=True, capture_output=True)

    def run(tuples):
        text = "\n".join(" ".join(repr(float(x)) for x in t) for t in tuples) + "\n"
        out = subprocess.run([str(exe)], input=text, capture_output=True, text=True, check=True).stdout
        return [tuple(int(x) for x in line.split()) for line in out.strip().splitlines()]

    return run


def test_keep_logic_on_every_weak_ordering(harness):
    table = json.load(open(os.path.join(GOLDEN, "topk_ties_m4.json")))["tables"]["2"]
    patterns = [row["pattern"] for row in table.values()]
    assert len(patterns) == 75
    for pat, (rel, keep, spread) in zip(patterns, harness(patterns)):
        want = table[[k for k, r in table.items() if r["pattern"] == pat][0]]["keep"]
        assert rel == want and keep == want, (pat, rel, keep, want)
        assert spread == sum(((want >> i) & 1) << (2 * i + 1) for i in range(4))


def test_keep_logic_on_a_grid_with_signed_zeros(harness):
    table = json.load(open(os.path.join(GOLDEN, "topk_ties_m4.json")))["tables"]["2"]
    levels = [-1.0, -0.0, 0.0, 0.25, 0.5, 1.0, 3.0]
    tuples = [(a, b, c, d) for a in levels for b in levels for c in levels for d in levels]
    for t, (rel, keep, spread) in zip(tuples, harness(tuples)):
        want = _torch_keep(t, table)  # -0.0 == +0.0 under < , as torch compares
        assert rel == want and keep == want, (t, rel, keep, want)
        assert bin(spread).count("1") == 2 and spread & 0x55 == 0
