"""Writes tests/golden/shuffle_order.json: the index orders std::shuffle produces over
std::iota(0..n) with a std::mt19937_64(seed) for three successive calls -- what the
reference's DataLoader does at construction and at each reset() (src/data/dataloader.cpp:
26-43).  The orders come from a small C++ program of this file, compiled with the system g++
(the standard library's own std::shuffle and std::mt19937_64)."""
import json
import os
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
PROGRAM = r"""
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <numeric>
#include <random>
#include <vector>
int main(int argc, char** argv) {
    const long n = std::atol(argv[1]);
    const unsigned long long seed = std::strtoull(argv[2], nullptr, 10);
    std::vector<int64_t> idx(n);
    std::iota(idx.begin(), idx.end(), int64_t{0});
    std::mt19937_64 rng(seed);
    for (int epoch = 0; epoch < 3; ++epoch) {
        std::shuffle(idx.begin(), idx.end(), rng);
        for (long i = 0; i < n; ++i) std::printf("%lld%c", static_cast<long long>(idx[i]), i + 1 < n ? ' ' : '\n');
    }
}
"""
CASES = [(28, 42), (23, 42), (1000, 7), (1, 42)]


def main():
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "s.cpp"), os.path.join(d, "s")
        open(src, "w").write(PROGRAM)
        subprocess.run(["g++", "-O1", "-std=c++17", src, "-o", exe], check=True)
        out = {}
        for n, seed in CASES:
            lines = subprocess.run([exe, str(n), str(seed)], check=True, capture_output=True, text=True).stdout
            out[f"{n}_{seed}"] = [[int(v) for v in l.split()] for l in lines.strip().splitlines()]
    with open(os.path.join(HERE, "shuffle_order.json"), "w") as f:
        json.dump(out, f)


if __name__ == "__main__":
    main()
