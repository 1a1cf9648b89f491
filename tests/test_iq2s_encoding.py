"""The IQ2_S device encoding (lightbridge-engine_amd/csrc/lbh_layout.h): a
bijection on the 82 block bytes, and the decode the kernels perform on it
(code-table address from one v_perm of the rotated qs dword and the spread qh
field, sign of weight 32g + 4k + i at bit k of byte i of the group's sign dword)
recovers the GGML block's grid index and sign of every weight
(crates/bridge-quant-layout/src/q8_k.rs:337-364: lookup l has grid index
qs[l] | ((qh[l / 4] >> 2 (l % 4)) & 3) << 8, and weight 8l + b the sign bit b of
sign byte l).

The header's host/device functions are compiled for the host with g++ and run
on random blocks and on the reference's own IQ2_S fixture block."""
import shutil
import subprocess

import numpy as np
import pytest

from pathlib import Path

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "lightbridge-engine_amd" / "csrc" / "lbh_layout.h"

CHECK = r"""
#define __host__
#define __device__
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include "lbh_layout.h"

static uint32_t u32(const uint8_t *p) { uint32_t v; std::memcpy(&v, p, 4); return v; }

// one block: round trip and the kernels' decode of the encoded bytes
static int check(const uint8_t *g) {
    uint8_t e[82], back[82];
    lbh::iq2s_encode(g, e);
    lbh::iq2s_decode(e, back);
    if (std::memcmp(g, back, 82)) return 1;
    if (e[0] != g[0] || e[1] != g[1] || std::memcmp(e + 74, g + 74, 8)) return 2;
    for (int grp = 0; grp < 8; ++grp) {
        const uint32_t q = u32(e + 2 + 4 * grp);            // rotated qs dword
        const uint32_t hw = u32(e + 66 + 4 * (grp / 4));     // qh dword of groups 4j .. 4j + 3
        const uint32_t s = u32(e + 34 + 4 * grp);            // sign dword
        const int k = grp & 3;
        const uint32_t hs = (k < 2 ? hw << (3 - 2 * k) : hw >> (2 * k - 3)) & 0x18181818u;
        const uint32_t x = q & 0xf8f8f8f8u, y = (q & 0x07070707u) | hs;
        for (int j = 0; j < 4; ++j) {
            const int l = 4 * grp + j;
            const uint32_t idx = g[2 + l] | (((g[66 + grp] >> (2 * j)) & 3u) << 8);
            const uint32_t addr = ((x >> (8 * j)) & 0xffu) + 256u * ((y >> (8 * j)) & 0xffu);
            if (addr != lbh::iq2s_code_addr_host(idx & 255u, idx >> 8)) return 3;
            for (int b = 0; b < 8; ++b) {
                const int w = 8 * j + b;                      // weight of the group
                const uint32_t want = (g[34 + l] >> b) & 1u;
                const int t = w / 4, i = w % 4;
                const uint32_t sel = (t >= 2 ? s >> (t - 2) : s << (2 - t)) & 0x04040404u;
                const uint32_t got = (sel >> (8 * i + 2)) & 1u;
                if (got != want) return 4;
            }
        }
    }
    return 0;
}

int main(int argc, char **argv) {
    // argv[1]: optional file of GGML blocks (82 bytes each)
    if (argc > 1) {
        FILE *f = std::fopen(argv[1], "rb");
        uint8_t g[82];
        int n = 0;
        while (std::fread(g, 1, 82, f) == 82) {
            const int r = check(g);
            if (r) { std::printf("fixture block %d: failure %d\n", n, r); return 1; }
            ++n;
        }
        std::fclose(f);
        std::printf("fixture blocks %d ok\n", n);
    }
    std::srand(7);
    for (int t = 0; t < 20000; ++t) {
        uint8_t g[82];
        for (int i = 0; i < 82; ++i) g[i] = (uint8_t)(std::rand() & 255);
        const int r = check(g);
        if (r) { std::printf("random block %d: failure %d\n", t, r); return 1; }
    }
    std::printf("random blocks ok\n");
    return 0;
}
"""

# Host twin of the device table address (lbh_dev.h iq2s_code_addr): byte
# address of code entry q | h << 8 in the 8 KiB table.
ADDR = r"""
namespace lbh {
inline uint32_t iq2s_code_addr_host(uint32_t q, uint32_t h) { return 256u * ((q >> 5) | (h << 3)) + 8u * (q & 31u); }
}
"""


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("no host C++ compiler")
    d = tmp_path_factory.mktemp("iq2s")
    src = d / "check.cpp"
    src.write_text(CHECK.replace('#include "lbh_layout.h"', '#include "lbh_layout.h"\n' + ADDR))
    exe = d / "check"
    subprocess.run([gxx, "-O2", "-std=c++17", f"-I{HEADER.parent}", str(src), "-o", str(exe)], check=True)
    return exe


def test_iq2s_encoding_random_blocks(checker):
    r = subprocess.run([str(checker)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "random blocks ok" in r.stdout


def test_iq2s_encoding_reference_fixture(checker, tmp_path):
    """The reference's IQ2_S fixture blocks (tests/golden/reference/decode-iq2-s.input.bin)."""
    blocks = sorted((REPO / "tests" / "golden" / "reference").glob("decode-iq2-s.input.bin"))
    assert blocks, "the reference's IQ2_S decode fixture is missing"
    assert all(p.stat().st_size % 82 == 0 for p in blocks)
    data = b"".join(p.read_bytes()[: (p.stat().st_size // 82) * 82] for p in blocks)
    f = tmp_path / "blocks.bin"
    f.write_bytes(data)
    r = subprocess.run([str(checker), str(f)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr


def test_iq2s_table_address_is_a_bijection():
    """Every 10-bit grid index gets its own 8-byte slot of the 8 KiB table."""
    q = np.arange(1024) & 255
    h = np.arange(1024) >> 8
    addr = 256 * ((q >> 5) | (h << 3)) + 8 * (q & 31)
    assert sorted(addr.tolist()) == list(range(0, 8192, 8))
