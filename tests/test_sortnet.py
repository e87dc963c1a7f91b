"""The device sorting network (gl-sdm_amd/csrc/sortnet16.h) sorts every input:
compiled on the host with g++ and checked on all 2^16 binary inputs (0-1 principle)."""
import os
import subprocess

from _util import ROOT

CHECK = r"""
#include <cstdio>
#include "sortnet16.h"
int main() {
    for (unsigned m = 0; m < (1u << 16); ++m) {
        int v[16];
        for (int i = 0; i < 16; ++i) v[i] = (m >> i) & 1;
        for (int c = 0; c < glsdm::SORTNET16_SIZE; ++c) {
            int a = glsdm::SORTNET16[c][0], b = glsdm::SORTNET16[c][1];
            if (v[a] > v[b]) { int t = v[a]; v[a] = v[b]; v[b] = t; }
        }
        for (int i = 0; i < 15; ++i) if (v[i] > v[i + 1]) { printf("fail %u\n", m); return 1; }
    }
    printf("ok\n");
    return 0;
}
"""


def test_sortnet16_sorts_all_binary_inputs(tmp_path):
    src = tmp_path / "check.cpp"
    exe = tmp_path / "check"
    src.write_text(CHECK)
    inc = os.path.join(ROOT, "gl-sdm_amd", "csrc")
    subprocess.run(["g++", "-O2", "-std=c++17", f"-I{inc}", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and out.stdout.strip() == "ok"
