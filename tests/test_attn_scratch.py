"""The attention scratch bound the model sizes its workspace with
(attention_scratch_bound, attn_plan.cpp) equals the brute-force maximum of
attention_scratch_floats over every (longest sequence, padded rows) pair it
stands for, on small and mid-size capacities of both head dims, with and
without a band.  The planning code is host arithmetic only; it is compiled
for the host and driven by a small C++ program (no GPU code, no device)."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "glypr_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"

DRIVER = r"""
#include <stdio.h>
#include "internal.hpp"
using namespace glypr;
static size_t brute(int64_t max_t, int64_t cap, int64_t nq, int64_t nkv, int64_t hd, int64_t w) {
  size_t best = 0;
  for (int64_t tk = 32;; tk += 32) {
    if (tk > max_t) tk = max_t;
    for (int64_t rows = attn_padded_len(tk); rows <= cap; rows += 64) {
      const size_t sc = attention_scratch_floats(tk, nq, nkv, hd, w, rows);
      best = sc > best ? sc : best;
    }
    if (tk == max_t) break;
  }
  return best;
}
int main() {
  const int64_t cases[][6] = {
      // max_t, cap, nq, nkv, hd, window
      {512, 512, 3, 1, 256, 512},     {1000, 4096, 3, 1, 256, 512},
      {2100, 8192, 3, 1, 256, 512},   {8320, 20480, 3, 1, 256, 512},
      {8320, 20480, 3, 1, 256, 0},    {8320, 32768, 4, 2, 256, 512},
      {4096, 16384, 4, 1, 512, 0},    {8320, 24576, 4, 1, 512, 0},
      {300, 65536, 3, 1, 256, 512},   {1536, 40960, 6, 2, 256, 128},
  };
  int bad = 0;
  for (const auto& c : cases) {
    const size_t a = attention_scratch_bound(c[0], c[1], c[2], c[3], c[4], c[5]);
    const size_t b = brute(c[0], c[1], c[2], c[3], c[4], c[5]);
    printf("%lld %lld %lld %lld %lld %lld: bound %zu brute %zu\n", (long long)c[0],
           (long long)c[1], (long long)c[2], (long long)c[3], (long long)c[4], (long long)c[5],
           a, b);
    bad += a != b;
  }
  return bad;
}
"""


def test_attention_scratch_bound_equals_brute_force(tmp_path):
    src = tmp_path / "scratch_check.cpp"
    src.write_text(DRIVER)
    exe = tmp_path / "scratch_check"
    common = ["-x", "hip", "--cuda-host-only", "-std=c++17", "-O2", f"-I{ROOT}/include",
              f"-I{CSRC}"]
    objs = []
    for path in (os.path.join(CSRC, "attn_plan.cpp"), str(src)):
        obj = str(tmp_path / (os.path.basename(path) + ".o"))
        r = subprocess.run([HIPCC, *common, "-c", path, "-o", obj], capture_output=True,
                           text=True)
        assert r.returncode == 0, r.stdout + r.stderr
        objs.append(obj)
    r = subprocess.run([HIPCC, "--cuda-host-only", *objs, "-o", str(exe)], capture_output=True,
                       text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
