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

}  // namespace lbh
