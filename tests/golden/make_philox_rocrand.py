"""Writes tests/golden/philox_rocrand.json: Philox4x32-10 outputs computed by
rocRAND's open-source implementation (/opt/rocm/include/rocrand/
rocrand_philox4x32_10.h, ten_rounds) on the host, for counters/keys that
exercise carries and the key schedule.  Run once; the JSON is the fixture."""
import json
import os
import subprocess
import tempfile

CASES = [([0, 0, 0, 0], [0, 0]), ([1, 0, 0, 0], [0, 0]), ([0, 0, 0, 0], [1, 0]),
         ([7, 3, 0, 0], [2, 0]), ([0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF], [0xFFFFFFFF, 0xFFFFFFFF]),
         ([15, 4, 2, 0], [0xDEADBEEF, 0x01234567]), ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344],
                                                     [0xA4093822, 0x299F31D0])]

SRC = r"""
#include <rocrand/rocrand_philox4x32_10.h>
#include <cstdio>
struct Engine : rocrand_device::philox4x32_10_engine {
  using rocrand_device::philox4x32_10_engine::ten_rounds;  // protected in the header
};
int main() {
  Engine e;
  unsigned v[6];
  while (scanf("%u %u %u %u %u %u", &v[0], &v[1], &v[2], &v[3], &v[4], &v[5]) == 6) {
    uint4 c = {v[0], v[1], v[2], v[3]};
    uint2 k = {v[4], v[5]};
    uint4 o = e.ten_rounds(c, k);
    printf("%u %u %u %u\n", o.x, o.y, o.z, o.w);
  }
}
"""

if __name__ == "__main__":
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "p.cpp")
        exe = os.path.join(d, "p")
        open(src, "w").write(SRC)
        subprocess.run(["hipcc", "-x", "hip", "--offload-arch=gfx950", "-I/opt/rocm/include", "-O1", src, "-o",
                        exe], check=True, capture_output=True)
        inp = "\n".join(" ".join(str(x) for x in c + k) for c, k in CASES) + "\n"
        out = subprocess.run([exe], input=inp, capture_output=True, text=True, check=True).stdout.split("\n")
    cases = [{"ctr": c, "key": k, "out": [int(x) for x in line.split()]} for (c, k), line in zip(CASES, out)]
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "philox_rocrand.json")
    json.dump({"source": "rocRAND rocrand_philox4x32_10.h ten_rounds (ROCm 7.2)", "cases": cases}, open(path, "w"),
              indent=1)
    print(f"wrote {path}")
