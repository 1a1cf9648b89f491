// lbh_layout.h — the device (HBM) layout of packed matrices.
//
// A GGML matrix of R rows x K columns has U = R * NB "units", one per
// (row, 256-element super-block), u = r * NB + b.  The device layout keeps
// exactly the same bytes (a lossless permutation, no padding) but splits each
// block into 16-byte chunks stored chunk-major:
//
//   chunk plane c : U x 16 B  at  c * U * 16 + u * 16        (c < NCHUNK)
//   tail plane    : U x TAIL  at  NCHUNK * U * 16 + u * TAIL  (IQ3_S only, 12 B)
//   d plane       : U x 2 B   at  NCHUNK * U * 16 + TAIL * U + u * 2 (IQ types)
//
// so a wave whose lanes own consecutive units issues fully coalesced
// 16-byte loads (1 KiB contiguous per instruction).  Inside a block:
//
//   IQ2_S (82 B)  chunks 0-1 qs[32], 2-3 signs[32], 4 qh[8]+scales[8]; d plane
//   IQ3_S (110 B) chunks 0-3 qs[64], 4-5 signs[32]; tail qh[8]+scales[4]; d plane
//   Q4_K (144 B)  chunk 0 d,dmin,scales[12]; chunks 1-8 qs[128] residue-major
//   Q5_K (176 B)  chunk 0 d,dmin,scales[12]; chunks 1-2 qh[32] residue-major;
//                 chunks 3-10 qs[128] residue-major
//
// "Residue-major": within every 32-byte group the byte at position l moves to
// 4 * (l % 8) + l / 8, so dword t of a group holds the four elements whose
// index is congruent to t mod 8 — the lane split of the reference K-quant dot
// (crates/bridge-quant-layout/src/q8_k.rs:301-312) becomes one dot4 per lane.
//
// IQ2_S blocks are stored bit-permuted inside their qs, sign and qh bytes (a
// bijection on the 82 bytes; d and the scales unchanged), so the decode of a
// group of 32 weights (four 8-weight lookups l = 4g + j, q8_k.rs:337-364)
// needs no per-lookup bit extraction:
//   qs byte l    the low 8 bits q of lookup l's grid index, rotated:
//                (q & 31) << 3 | q >> 5.  With the lookup's two high bits h at
//                bits 3-4 of a byte, (rotated & 0xf8) + 256 * ((rotated & 7) |
//                h << 3) is a byte address of an 8 KiB table (one v_perm for a
//                lookup, the qs dword supplying four);
//   qh dword j   (bytes 4j..4j+3 of the qh bytes) byte j', bits 2k, 2k + 1:
//                the high bits of lookup j' of group 4j + k (a 4 x 4 transpose
//                of the 2-bit fields of qh[4j..4j+3]);
//   sign dword g (sign bytes 4g..4g+3) byte i, bit k: the sign of weight
//                32g + 4k + i, so the four signs of weights 32g + 4k .. + 3 sit
//                at bit k of consecutive bytes (one shift and mask give the
//                v_perm selector bits that apply them).
#pragma once
#include <stdint.h>

namespace lbh {

enum : int { T_F32 = 0, T_Q4_K = 12, T_Q5_K = 13, T_Q8_K = 15, T_IQ3_S = 21, T_IQ2_S = 22 };

struct TypeLayout {
    int block_bytes;
    int nchunk;    // 16-byte chunks per unit
    int tail;      // tail-plane bytes per unit
    int dplane;    // 1: f16 d stored in its own plane
};

__host__ __device__ constexpr TypeLayout layout_of(int ty) {
    return ty == T_IQ2_S   ? TypeLayout{82, 5, 0, 1}
           : ty == T_IQ3_S ? TypeLayout{110, 6, 12, 1}
           : ty == T_Q4_K  ? TypeLayout{144, 9, 0, 0}
           : ty == T_Q5_K  ? TypeLayout{176, 11, 0, 0}
                           : TypeLayout{0, 0, 0, 0};
}

__host__ __device__ constexpr bool is_dot_type(int ty) {
    return ty == T_IQ2_S || ty == T_IQ3_S || ty == T_Q4_K || ty == T_Q5_K;
}

// Position of byte l (0..31) of a 32-byte group in residue-major order.
__host__ __device__ constexpr int residue_pos(int l) { return 4 * (l % 8) + l / 8; }

// IQ2_S block bytes: d 0-1, qs 2-33, signs 34-65, qh 66-73, scales 74-81.
__host__ __device__ constexpr uint8_t iq2s_rot_q(uint32_t q) { return (uint8_t)(((q & 31u) << 3) | (q >> 5)); }
__host__ __device__ constexpr uint8_t iq2s_unrot_q(uint32_t r) { return (uint8_t)((r >> 3) | ((r & 7u) << 5)); }

// GGML bytes g of one IQ2_S block -> its device encoding e (82 bytes each).
__host__ __device__ inline void iq2s_encode(const uint8_t *g, uint8_t *e) {
    e[0] = g[0], e[1] = g[1];
    for (int l = 0; l < 32; ++l) e[2 + l] = iq2s_rot_q(g[2 + l]);
    for (int grp = 0; grp < 8; ++grp)
        for (int i = 0; i < 4; ++i) {
            uint32_t v = 0;
            for (int k = 0; k < 8; ++k) v |= ((uint32_t)(g[34 + 4 * grp + (k >> 1)] >> (4 * (k & 1) + i)) & 1u) << k;
            e[34 + 4 * grp + i] = (uint8_t)v;
        }
    for (int j = 0; j < 2; ++j)
        for (int jj = 0; jj < 4; ++jj) {
            uint32_t v = 0;
            for (int k = 0; k < 4; ++k) v |= ((uint32_t)(g[66 + 4 * j + k] >> (2 * jj)) & 3u) << (2 * k);
            e[66 + 4 * j + jj] = (uint8_t)v;
        }
    for (int s = 74; s < 82; ++s) e[s] = g[s];
}

// The inverse of iq2s_encode.
__host__ __device__ inline void iq2s_decode(const uint8_t *e, uint8_t *g) {
    g[0] = e[0], g[1] = e[1];
    for (int l = 0; l < 32; ++l) g[2 + l] = iq2s_unrot_q(e[2 + l]);
    for (int grp = 0; grp < 8; ++grp)
        for (int jj = 0; jj < 4; ++jj) {
            uint32_t v = 0;
            for (int b = 0; b < 8; ++b) v |= ((uint32_t)(e[34 + 4 * grp + (b & 3)] >> (2 * jj + (b >> 2))) & 1u) << b;
            g[34 + 4 * grp + jj] = (uint8_t)v;
        }
    for (int j = 0; j < 2; ++j)
        for (int k = 0; k < 4; ++k) {
            uint32_t v = 0;
            for (int jj = 0; jj < 4; ++jj) v |= ((uint32_t)(e[66 + 4 * j + jj] >> (2 * k)) & 3u) << (2 * jj);
            g[66 + 4 * j + k] = (uint8_t)v;
        }
    for (int s = 74; s < 82; ++s) g[s] = e[s];
}

}  // namespace lbh
