"""Writes libstdcxx_uniform.json: draws of std::mt19937 and of
std::uniform_real_distribution<double> as this machine's libstdc++ computes
them, the generator the reference's SpMMOp tests use for their matrices
(test/spmm_op/spmm_op_golden.h:104-121, test/spmm_op/arch35/spmm_op_test.cpp:121-133).

The vectors come from a small C++ program compiled here with g++ against the
standard library only (no reference code).  They pin oracle.mt19937 and
oracle.uniform_real, the restatement the tests use to rebuild the reference's
exact inputs.

Run: python tests/golden/make_libstdcxx_vectors.py
"""
import json
import os
import subprocess
import tempfile

H = os.path.dirname(os.path.abspath(__file__))

PROGRAM = r"""
#include <cstdio>
#include <random>
int main() {
    const unsigned seeds[] = {0u, 1u, 2u, 101u, 5489u, 20260909u, 4294967295u};
    const double ranges[][2] = {{-1.0, 1.0}, {-0.5, 0.5}, {-3.0, 3.0}, {0.0, 1.0}};
    std::printf("{\"raw\": [");
    for (int s = 0; s < 7; ++s) {
        std::mt19937 g(seeds[s]);
        std::printf("%s{\"seed\": %u, \"words\": [", s ? ", " : "", seeds[s]);
        for (int i = 0; i < 700; ++i) std::printf("%s%u", i ? ", " : "", (unsigned)g());
        std::printf("]}");
    }
    std::printf("], \"uniform\": [");
    int first = 1;
    for (int s = 0; s < 7; ++s) {
        for (int r = 0; r < 4; ++r) {
            std::mt19937 g(seeds[s]);
            std::uniform_real_distribution<double> d(ranges[r][0], ranges[r][1]);
            std::printf("%s{\"seed\": %u, \"lo\": %.17g, \"hi\": %.17g, \"values\": [", first ? "" : ", ", seeds[s],
                        ranges[r][0], ranges[r][1]);
            first = 0;
            for (int i = 0; i < 400; ++i) std::printf("%s%.17g", i ? ", " : "", d(g));
            std::printf("]}");
        }
    }
    std::mt19937 def;
    unsigned long long v = 0;
    for (int i = 0; i < 10000; ++i) v = def();
    std::printf("], \"default_10000th\": %llu}\n", v);
    return 0;
}
"""


def main():
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "gen.cpp")
        exe = os.path.join(d, "gen")
        open(src, "w").write(PROGRAM)
        subprocess.run(["g++", "-O1", "-std=c++17", src, "-o", exe], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    data = json.loads(out)
    data["generator"] = "g++ " + subprocess.run(["g++", "-dumpfullversion"], capture_output=True,
                                                text=True).stdout.strip() + " libstdc++"
    with open(os.path.join(H, "libstdcxx_uniform.json"), "w") as f:
        json.dump(data, f)


if __name__ == "__main__":
    main()
