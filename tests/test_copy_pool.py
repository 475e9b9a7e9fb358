"""The host entries' copy threads (picolm_qwen_amd/csrc/pqa_copy_pool.h), built
on the CPU with g++: every byte of [0, n) copied and nothing past it, for 0 to 7
worker threads and sizes that do not divide evenly into the threads' pieces
(with 7 workers and 8 pieces, n = 512 m + 4 once lost its last 4 bytes)."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SRC = r"""
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>
#include "pqa_copy_pool.h"

int main() {
    const size_t MiB = size_t(1) << 20;
    std::vector<size_t> sizes = {0, 1, 4, 1000, MiB - 4, MiB, MiB + 4, 8 * MiB, 8 * MiB + 3};
    for (size_t parts = 1; parts <= 8; ++parts)
        for (size_t r = 1; r < parts; ++r) sizes.push_back(parts * 64 * 4096 + r);  // share a multiple of 64
    for (size_t k = 0; k < 24; ++k) sizes.push_back(MiB + 977 * k * k * k + 13 * k);
    const size_t guard = 256;
    for (int workers = 0; workers <= 7; ++workers) {
        pqa::CopyPool pool(workers);
        for (size_t n : sizes) {
            std::vector<unsigned char> src(n + guard), dst(n + guard, 0xEE);
            for (size_t i = 0; i < src.size(); ++i) src[i] = (unsigned char)(i * 131 + (i >> 8) + workers);
            pool.copy((char*)dst.data(), (const char*)src.data(), n);
            if (std::memcmp(dst.data(), src.data(), n) != 0) {
                std::printf("workers %d n %zu: bytes differ\n", workers, n);
                return 1;
            }
            for (size_t i = n; i < n + guard; ++i)
                if (dst[i] != 0xEE) {
                    std::printf("workers %d n %zu: byte %zu past the end written\n", workers, n, i);
                    return 1;
                }
        }
    }
    std::printf("ok\n");
    return 0;
}
"""


def test_copy_pool_copies_every_byte_and_no_more(tmp_path):
    src = tmp_path / "copy_pool_check.cpp"
    src.write_text(SRC)
    exe = tmp_path / "copy_pool_check"
    subprocess.run(["g++", "-std=c++17", "-O2", "-pthread", "-I", os.path.join(ROOT, "picolm_qwen_amd", "csrc"),
                    str(src), "-o", str(exe)], check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and out.stdout.strip() == "ok", out.stdout + out.stderr
