// Staging of bf16 operand tiles into LDS for the MFMA kernels (gfx950):
// direct memory-to-LDS transfers (buffer_load ... lds) and the transposing
// fragment read ds_read_b64_tr_b16, plus the swizzled layout of a tile of
// 512-byte rows that both are used with.
#pragma once

#include "common.h"

typedef __attribute__((address_space(3))) uint8_t lds_u8_t;
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

// A buffer resource as four scalar words (base, stride 0, size in bytes,
// flags), the layout __builtin_amdgcn_make_buffer_rsrc builds, for inline
// assembly.  With stride 0 the range check compares the VGPR offset (not the
// scalar offset) with the size: a transfer at or past it reads zeros.
DPC_DEVICE u32x4_t rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return u32x4_t{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, bytes, 0x00020000u};
}

// buffer_load_dwordx4 ... lds: lane i's 16 bytes at buffer offset voff + soff
// go to LDS address lds + 16 i.  Inline assembly, so that the compiler does
// not see an LDS write: it would otherwise make the fragment reads of the
// other stages wait for every transfer in flight.  The caller orders the
// transfers with explicit memory-counter waits (DPC_WAIT_VMCNT) and barriers.
DPC_DEVICE void dma16(u32x4_t rsrc, uint32_t lds, int voff, int soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds), "v"(voff), "s"(rsrc), "s"(soff)
               : "m0");
}

// buffer_load_dword ... lds: lane i's 4 bytes go to LDS address lds + 4 i.
DPC_DEVICE void dma4(u32x4_t rsrc, uint32_t lds, int voff, int soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, %3 offen lds"
               :
               : "s"(lds), "v"(voff), "s"(rsrc), "s"(soff)
               : "m0");
}

DPC_DEVICE uint32_t lds_addr(const uint8_t* p) {
  return (uint32_t)reinterpret_cast<uintptr_t>((const lds_u8_t*)p);
}

// Transposing read of 4 k-consecutive bf16 per lane (ds_read_b64_tr_b16):
// lane L of a 16-lane group supplies the address of 4 consecutive columns of
// one row, and after the read holds column L of the group's 4 rows.
DPC_DEVICE i16x4_t read_tr(const uint8_t* lds_base, int off) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4_t*)((__attribute__((address_space(3))) uint8_t*)lds_base + off));
}

DPC_DEVICE bf16x8_t join_frag(i16x4_t lo, i16x4_t hi) {
  return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// ---------------------------------------------------------------------------
// A tile of k rows of 256 bf16 (512 bytes): the row's eight 64-byte blocks
// permuted by XOR with (k & 7), and the two 32-byte halves of every block
// swapped in rows with bit 2 of k set.  The 64 four-byte banks span 256
// bytes, so blocks b and b ^ 4 of a row share banks.  A 16-lane group of a
// 16-byte store covers 4 consecutive blocks of one row, and a 32-lane half of
// a fragment read (frag16_off) covers one 32-byte half block in 8 rows
// (k & 7 = 0 .. 7, the rows with bit 2 set in the other half): both land on
// 64 distinct banks.
// ---------------------------------------------------------------------------
constexpr int kTileRowBytes = 512;

// Byte offset of bf16 element (k, col) (col < 256; 16-byte chunks of 8
// columns stay contiguous).
DPC_DEVICE int tile_off(int k, int col) {
  return k * kTileRowBytes +
         ((((col >> 5) ^ (k & 7)) << 6) | (((col & 31) << 1) ^ (((k >> 2) & 1) << 5)));
}

// Logical first column of the 16-byte chunk at physical 16-byte slot `slot`
// (0..31) of row k: the inverse of tile_off.
DPC_DEVICE int tile_slot_col(int k, int slot) {
  return (((slot >> 2) ^ (k & 7)) << 5) + (((slot & 3) ^ (((k >> 2) & 1) << 1)) << 3);
}

// Per-lane LDS offset of the transposing fragment read for a 16 x 32
// fragment of the 16x16x32 MFMA at tile column c0, K sub-step 0, half h
// (k-slots 4h..4h+3 of the lane's 8).  The MFMA operand lane l holds k-slots
// 8 (l / 16) .. + 7 of row (column) l % 16.  The k-slots are a permutation of
// the sub-step's 32 rows, the same for both operands, so the MFMA still sums
// over all of them: slot 8 q + 4 h + e (q = l / 16, e < 4) is row 16 h + 4 q
// + e.  Lane L of group q reads the 8 bytes at k = 16 h + 4 q + (L >> 2),
// col = c0 + 4 (L & 3), and after the transpose holds 4 consecutive rows of
// col c0 + L.  With this order the two 16-lane groups of a 32-lane half read
// rows 4 q' .. 4 q' + 3 and 4 q' + 4 .. 4 q' + 7: 8 distinct (k & 7), the
// second four with swapped block halves, which is what keeps the read on 64
// distinct banks (tile_off).  Sub-step kk adds kk * 32 rows.
DPC_DEVICE int frag16_off(int c0, int h, int lane) {
  const int q = lane >> 4, L = lane & 15;
  return tile_off(16 * h + 4 * q + (L >> 2), c0 + 4 * (L & 3));
}
