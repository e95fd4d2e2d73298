// The gfx950 tile layout of packed weight matrices, shared by the host repacker and the kernels.
//
// A matrix of R packed rows (outputs, R % 16 == 0) and K columns (K % 128 == 0) is cut into tiles of 16 rows and
// groups of 128 columns; tile t, group g is one contiguous block, blocks ordered [t][g] so that a wave walking the
// groups of its tiles streams contiguous memory.
//
// The block holds exactly the B operand of v_mfma_f32_16x16x32_bf16 (B = W^T, 32 k x 16 outputs) for the group's
// four k32 steps j = 0..3: lane l (0..63) owns output row 16t + l % 16 and the 8 columns
// k = 128g + 32j + 8(l / 16) + 0..7 of each step.
//
//  int4 (QH_WT_I4, QH_WT_I4Z): 1024 B per block = [lane][j] u32 — a lane reads its four steps with one 16-byte load
//    and a wave reads the block as one contiguous KiB. In a word the 8 columns c = 0..7 sit in nibble position
//    c / 2 for even c and 4 + c / 2 for odd c, so that (word >> 4p) & 0x000F000F holds columns 2p (low half) and
//    2p + 1 (high half): one and-or with 0x43004300 turns them into the bf16 pair (128 + q, 128 + q').
//    Stored values are the checkpoint's unsigned codes (q + 8 of a symmetric value).
//  int8 (QH_WT_I8): 2048 B per block = [h][lane][w] u32, h = 0, 1: words w = 2e + i, step j = 2h + e, column bytes
//    4i + 0..3 in byte order; stored values q + 128.
//  bf16 (QH_WT_BF16, dense 16-bit weights): 4096 B per block = [j][lane] 16 bytes, the lane's 8 columns of step j as
//    bf16 in column order, so that each 16-byte piece is a B fragment as loaded. No scales or zero points.
//
// Scales: per quad of 4 groups (the group count padded up to a multiple of 4), per tile, per row of the tile, the
// quad's 4 groups: [g / 4][t][16][g % 4] (T tiles), so that one 8-byte load gives a row the scales of 4 consecutive
// groups, and the tiles of one quad, which the decode kernel's concurrently running workgroups read together, are one
// contiguous run. bf16 for int4 (exact for bf16-stored checkpoint scales), f32 for int8 and for the int4 _S32
// storages (scales bf16 does not hold exactly).
// Zero points (QH_WT_I4Z, QH_WT_I4Z_S32): [g / 4][t][16] u16, nibble g % 4 = the zero point of that row and group.
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace qh {

constexpr int TILE = 16;   // rows per tile
constexpr int QG = 128;    // columns per group (one scale, one zero point)
constexpr int LANES = 64;  // wavefront size

// storage properties (enum qh_wt values)
constexpr bool is_i8(int wt) { return wt == 1; }
constexpr bool is_bf16(int wt) { return wt == 6; }
constexpr bool has_zeros(int wt) { return wt == 3 || wt == 5; }
constexpr bool has_scales(int wt) { return !is_bf16(wt); }
constexpr bool f32_scales(int wt) { return wt == 1 || wt == 4 || wt == 5; }
constexpr bool valid_wt(int wt) { return wt >= 1 && wt <= 6; }

// bytes of one (tile, group) code block
constexpr size_t block_bytes(int wt) { return is_bf16(wt) ? 4096 : is_i8(wt) ? 2048 : 1024; }

// quads of 4 groups (scale and zero-point blocks) for G groups
constexpr size_t quads(size_t G) { return (G + 3) / 4; }
// element index of the scale of tile t, group g, row r (T tiles in the matrix)
constexpr size_t scale_idx(size_t t, size_t T, size_t g, int r) {
    return (((g / 4) * T + t) * TILE + (size_t)r) * 4 + g % 4;
}
// u16 index of the zero-point nibbles of tile t, quad g / 4, row r (T tiles)
constexpr size_t zero_idx(size_t t, size_t T, size_t g, int r) { return ((g / 4) * T + t) * TILE + (size_t)r; }

// nibble position of column c (0..7) inside a packed int4 word
constexpr int nib_pos(int c) { return (c & 1) ? 4 + (c >> 1) : (c >> 1); }

}  // namespace qh
