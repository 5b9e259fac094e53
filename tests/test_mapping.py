"""CPU check of the causal work-group order (trainium-linear-attention_amd/csrc/la_internal.hpp
map_causal_block): the header itself is compiled for the host with hipcc, and for many grids the
map must be a bijection from work-group ids onto (head, query block) pairs, with or without the
paired first round (pair_cus > 0), each XCD (work-group id mod 8) owning whole heads when the head
count is a multiple of 8, and every XCD's work-groups ordered heaviest block first outside the
reversed half of the first round."""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "trainium-linear-attention_amd", "csrc")

PROGRAM = r"""
#include <cstdio>
#include <vector>
#include "la_internal.hpp"

int main() {
  const int bhs[] = {1, 2, 3, 4, 7, 8, 16, 24, 32, 64, 128};
  const int nqbs[] = {1, 2, 3, 5, 8, 16, 31, 32, 64, 100};
  const int pairs[] = {0, 1, 4, 32};
  long checked = 0;
  for (int BH : bhs)
    for (int nqb : nqbs)
      for (int pc : pairs) {
        std::vector<int> seen((size_t)BH * nqb, 0);
        std::vector<int> last_qb(8, 1 << 30);
        const int T = (BH & 7) == 0 ? (BH / 8) * nqb : 0;
        for (int wg = 0; wg < BH * nqb; ++wg) {
          int bh = -1, qb = -1;
          la::map_causal_block(wg, BH, nqb, bh, qb, pc);
          if (bh < 0 || bh >= BH || qb < 0 || qb >= nqb) {
            printf("FAIL range BH=%d nqb=%d pc=%d wg=%d -> (%d, %d)\n", BH, nqb, pc, wg, bh, qb);
            return 1;
          }
          if (seen[(size_t)bh * nqb + qb]++) {
            printf("FAIL twice BH=%d nqb=%d pc=%d (%d, %d)\n", BH, nqb, pc, bh, qb);
            return 1;
          }
          if ((BH & 7) == 0) {
            const int x = wg & 7, s = wg >> 3;
            if (bh % 8 != x) {
              printf("FAIL xcd BH=%d nqb=%d pc=%d wg=%d bh=%d\n", BH, nqb, pc, wg, bh);
              return 1;
            }
            const bool reversed = pc > 0 && T >= 2 * pc && s >= pc && s < 2 * pc;
            if (!reversed) {
              if (qb > last_qb[x]) {
                printf("FAIL order BH=%d nqb=%d pc=%d wg=%d qb=%d\n", BH, nqb, pc, wg, qb);
                return 1;
              }
              last_qb[x] = qb;
            } else if (s == 2 * pc - 1) {
              // after the reversed half the order continues from the heaviest block it left
              last_qb[x] = nqb - 1 - (2 * pc - 1) / (BH / 8);
            }
          }
          ++checked;
        }
      }
  printf("OK %ld\n", checked);
  return 0;
}
"""


def test_map_causal_block_is_a_bijection(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    src = tmp_path / "mapping.hip"
    src.write_text(PROGRAM)
    exe = tmp_path / "mapping"
    r = subprocess.run([hipcc, "-O1", "-std=c++17", "--offload-arch=gfx950", "-I", CSRC, str(src), "-o", str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    print(out.stdout.strip())
    assert out.returncode == 0 and out.stdout.startswith("OK"), out.stdout + out.stderr
