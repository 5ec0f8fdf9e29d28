// fms_device.hpp -- gfx950 device building blocks shared by every MaxSim scan.
//
// Tiling (CDNA4, wave64):
//   One MFMA 32x32xK instruction per k-block multiplies a 32-token document
//   chunk (A operand: row i = document token) by a 32-token query tile
//   (B operand: column j = query token).  The fp32/int32 result lives in 16
//   accumulator registers per lane:
//       lane l, register r  <->  row 8*(r/4) + 4*(l/32) + r%4,  column l%32
//   so every lane owns ONE query token (column) and 16 document tokens of
//   the chunk, and the per-query-token running max / argmax is a private
//   per-lane scan; lanes l and l^32 are merged once per (pair, query tile).
//
// Operand fragments: lane l supplies row/column l%32 and k-slots
//   [kb*KB + (l/32)*EPL, +EPL) of k-block kb.  The same slot mapping is used
//   for A and B, so each MFMA sums whole dot products over its KB k values.
//
// Loads go through raw buffer resources (one per document / query / mask),
// which makes every read past the end of a sequence return zero instead of
// touching memory: ragged tails need no guards and cannot fault.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace fms {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kTile = 32;      // query tokens per tile == document tokens per chunk
constexpr int kWaves = 4;      // waves per workgroup for the scan kernels
constexpr int kRsrcWord3 = 0x00020000;  // gfx9-family raw buffer descriptor word 3

typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcWord3);
}

// Resource whose base and size are forced into scalar registers.  Every
// sequence a wave reads is uniform across the wave; when the compiler
// cannot prove that for a loop-carried value it builds the descriptor in
// vector registers and wraps each load in a waterfall loop, which also
// defeats the in-order vmcnt accounting the prefetch relies on.
// Wave-uniform copies of 32- / 64-bit values.  __builtin_amdgcn_readfirstlane
// returns a signed int: it must become uint32_t before any widening, or a
// low word with bit 31 set sign-extends into the high word.
__device__ __forceinline__ uint32_t rfl32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)v);
}
__device__ __forceinline__ uint64_t rfl64(uint64_t v) {
  return ((uint64_t)rfl32((uint32_t)(v >> 32)) << 32) | (uint64_t)rfl32((uint32_t)v);
}

__device__ __forceinline__ rsrc_t make_rsrc_u(const void* base, uint32_t bytes) {
  return make_rsrc(reinterpret_cast<const void*>(rfl64(reinterpret_cast<uint64_t>(base))),
                   rfl32(bytes));
}

__device__ __forceinline__ u32x4 buf_load16(rsrc_t r, int voff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
}
// Four fp32 values.  Bit-cast the whole 128-bit result before extracting
// lanes: extracting i32 elements first and bit-casting each to float makes
// this compiler (ROCm 7.2 clang, -O3) shrink the load to a single dword and
// broadcast it to all four elements.
__device__ __forceinline__ f32x4 buf_load16f(rsrc_t r, int voff) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
}
__device__ __forceinline__ uint32_t buf_load4(rsrc_t r, int voff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, 0, 0);
}
__device__ __forceinline__ uint32_t buf_load2(rsrc_t r, int voff) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, voff, 0, 0);
}
__device__ __forceinline__ uint32_t buf_load1(rsrc_t r, int voff) {
  return __builtin_amdgcn_raw_buffer_load_b8(r, voff, 0, 0);
}

// ---- MFMA operand traits ------------------------------------------------------
// kEsz: bytes per stored element; kEpl: elements per lane per k-block;
// kKb: k values per MFMA (two lane halves x kEpl); Frag: raw register image
// of one lane's operand; Acc: 16-register accumulator.

struct OpF16 {
  static constexpr int kEsz = 2, kEpl = 8, kKb = 16;
  static constexpr bool kInt = false;
  typedef u32x4 Frag;
  typedef f32x16 Acc;
  __device__ static Frag zero() { return u32x4{0u, 0u, 0u, 0u}; }
  __device__ static Frag load(rsrc_t r, int voff) { return buf_load16(r, voff); }
  __device__ static Acc mma(Frag a, Frag b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  // Element-wise guarded load (dim not a multiple of kEpl): elements with
  // k >= dim are zero.  `voff` addresses element k0 of the row.
  __device__ static Frag load_guarded(rsrc_t r, int voff, int k0, int dim) {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      uint32_t lo = (k0 + 2 * e < dim) ? buf_load2(r, voff + 4 * e) : 0u;
      uint32_t hi = (k0 + 2 * e + 1 < dim) ? buf_load2(r, voff + 4 * e + 2) : 0u;
      w[e] = (lo & 0xffffu) | (hi << 16);
    }
    return u32x4{w[0], w[1], w[2], w[3]};
  }
};

struct OpBF16 : OpF16 {
  __device__ static Acc mma(Frag a, Frag b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

// INT8 codes; kDsHalf: the document scales are stored as fp16 (an
// Int8Index quantised from Float16 features keeps Float16 scales) rather
// than fp32.  Both widen exactly to fp32 before the dequant.
template <bool kDsHalf_>
struct OpI8T {
  static constexpr int kEsz = 1, kEpl = 16, kKb = 32;
  static constexpr bool kInt = true;
  static constexpr bool kDsHalf = kDsHalf_;
  typedef u32x4 Frag;
  typedef i32x16 Acc;
  __device__ static Frag zero() { return u32x4{0u, 0u, 0u, 0u}; }
  __device__ static Frag load(rsrc_t r, int voff) { return buf_load16(r, voff); }
  __device__ static Acc mma(Frag a, Frag b, Acc c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a),
                                                 __builtin_bit_cast(i32x4, b), c, 0, 0, 0);
  }
  __device__ static Frag load_guarded(rsrc_t r, int voff, int k0, int dim) {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      uint32_t acc = 0u;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        uint32_t v = (k0 + 4 * e + b < dim) ? buf_load1(r, voff + 4 * e + b) : 0u;
        acc |= (v & 0xffu) << (8 * b);
      }
      w[e] = acc;
    }
    return u32x4{w[0], w[1], w[2], w[3]};
  }
};
typedef OpI8T<false> OpI8;   // fp32 document scales
typedef OpI8T<true> OpI8H;   // fp16 document scales

struct OpF32 {
  static constexpr int kEsz = 4, kEpl = 1, kKb = 2;
  static constexpr bool kInt = false;
  typedef uint32_t Frag;
  typedef f32x16 Acc;
  __device__ static Frag zero() { return 0u; }
  __device__ static Frag load(rsrc_t r, int voff) { return buf_load4(r, voff); }
  __device__ static Acc mma(Frag a, Frag b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(__builtin_bit_cast(float, a),
                                                __builtin_bit_cast(float, b), c, 0, 0, 0);
  }
  __device__ static Frag load_guarded(rsrc_t r, int voff, int k0, int dim) {
    return (k0 < dim) ? buf_load4(r, voff) : 0u;
  }
};

// Document row (within a 32-token chunk) held by accumulator register r of
// a lane in half h (= lane / 32).
__device__ __forceinline__ constexpr int acc_row(int r, int h) {
  return 8 * (r >> 2) + 4 * h + (r & 3);
}

// Running (max, slot) update over one chunk's 16 scores of this lane;
// slot = chunk*16 + r identifies (chunk, register) until the final merge.
// Registers ascend in document row within a wave half (acc_row), so the
// reference's sequential rule -- first valid token wins, then only a
// strictly greater score replaces (forward_pair.jl:82-85) -- is: the
// chunk's maximum with the LOWEST register among equal maxima, merged into
// the running max only if strictly greater (earlier chunks win ties).
//
// fold_tree: a v_max3 tree gives the chunk maximum, a reverse scan the first
// register equal to it -- short dependency chains, ~2.6 VALU ops per score.
// Every row must hold a valid token (callers substitute masked rows).
//
// The maxima are IEEE 754-2019 maximumNumber: a NaN operand is ignored, so
// NaN scores never become the chunk maximum -- as NaN never compares greater
// in the reference's `s > mx`.  That is what v_max3_f32 does in the IEEE
// mode compute kernels run in, and the compiler emits it for these chains
// (with the occasional input canonicalisation).  It must stay compiler
// visible: the tree's operands are MFMA results, and the compiler inserts
// the wait states an MFMA result needs before a VALU reads it only for
// instructions it can see -- an inline-asm v_max3 placed right after the
// MFMAs read accumulators that were not yet written.  Written as
// max(max(a, b), c) and with every node of the tree a three-input max (the
// root's third input -inf), the chains lower to v_max3_f32 alone; a lone
// two-input max over MFMA results would get an input canonicalisation per
// operand.  (A chunk whose scores are all NaN then has maximum -inf instead
// of NaN; neither is ever strictly greater than the running max.)
__device__ __forceinline__ float max3_ieee(float a, float b, float c) {
  return __builtin_fmaximum_numf(__builtin_fmaximum_numf(a, b), c);
}

// Three steps of the reverse scan for the first register equal to the
// chunk maximum: ci = R2 if x2 == cm, else R1 if x1 == cm, else R0 if
// x0 == cm, else ci (x0, x1, x2 are registers R0 > R1 > R2, scanned in that
// order).  A compare writes its lane mask to an SGPR pair, and gfx950 needs
// two wait states between a VALU write of an SGPR and a VALU read of it;
// the compiler routes every compare of the scan through VCC and so pads
// each select with an s_nop.  Here the three compares go to three SGPR
// pairs and each select reads its mask three instructions later, with no
// padding.  The operands are MFMA results, but every caller's
// compiler-visible max3 tree has read all of them before cm exists, so the
// MFMA-result wait states are already behind (see max3_ieee).
template <int R0, int R1, int R2>
__device__ __forceinline__ void first_equal3(int& ci, float x0, float x1, float x2, float cm) {
  uint64_t e0, e1, e2;
  asm("v_cmp_eq_f32_e64 %1, %4, %7\n\t"
      "v_cmp_eq_f32_e64 %2, %5, %7\n\t"
      "v_cmp_eq_f32_e64 %3, %6, %7\n\t"
      "v_cndmask_b32_e64 %0, %0, %8, %1\n\t"
      "v_cndmask_b32_e64 %0, %0, %9, %2\n\t"
      "v_cndmask_b32_e64 %0, %0, %10, %3"
      : "+v"(ci), "=&s"(e0), "=&s"(e1), "=&s"(e2)
      : "v"(x0), "v"(x1), "v"(x2), "v"(cm), "n"(R0), "n"(R1), "n"(R2));
}

// kPadFree: the reverse scan as first_equal3 blocks (no wait-state
// padding).  Those blocks are opaque to the scheduler, which then cannot
// spread a tile's fold between the MFMAs of the next tiles as it does with
// the compiler's own compares; the in-batch kernel, whose throughput rests
// on that interleave, keeps the compiler's form.
// kRowSlots: the slot records the register's row offset acc_row(r, 0)
// instead of r (slot0 + acc_row(r, 0) + 4 h is then the chunk row), so a
// close turns a slot into a token with one add.  Both are compile-time
// constants of the scan.
template <bool kRowSlots>
__device__ __forceinline__ constexpr int reg_slot(int r) {
  return kRowSlots ? acc_row(r, 0) : r;
}

// first_equal3 over registers r0, r0 - 1, r0 - 2 of a chunk's scores.
template <bool kRowSlots, int kR0>
__device__ __forceinline__ void first_equal_regs(int& ci, const float (&s)[16], float cm) {
  first_equal3<reg_slot<kRowSlots>(kR0), reg_slot<kRowSlots>(kR0 - 1), reg_slot<kRowSlots>(kR0 - 2)>(
      ci, s[kR0], s[kR0 - 1], s[kR0 - 2], cm);
}

template <bool kPadFree, bool kRowSlots = false>
__device__ __forceinline__ void fold_tree(const float (&s)[16], int slot0, float& mx, int& slot) {
  const float m0 = max3_ieee(s[0], s[1], s[2]);
  const float m1 = max3_ieee(s[3], s[4], s[5]);
  const float m2 = max3_ieee(s[6], s[7], s[8]);
  const float m3 = max3_ieee(s[9], s[10], s[11]);
  const float m4 = max3_ieee(s[12], s[13], s[14]);
  const float m5 = max3_ieee(s[15], m0, m1);
  const float m6 = max3_ieee(m2, m3, m4);
  const float cm = max3_ieee(m5, m6, -INFINITY);
  int ci = reg_slot<kRowSlots>(15);
  if constexpr (kPadFree) {
    first_equal_regs<kRowSlots, 14>(ci, s, cm);
    first_equal_regs<kRowSlots, 11>(ci, s, cm);
    first_equal_regs<kRowSlots, 8>(ci, s, cm);
    first_equal_regs<kRowSlots, 5>(ci, s, cm);
    first_equal_regs<kRowSlots, 2>(ci, s, cm);
  } else {
#pragma unroll
    for (int r = 14; r >= 0; --r) ci = (s[r] == cm) ? reg_slot<kRowSlots>(r) : ci;
  }
  const bool take = cm > mx;
  mx = take ? cm : mx;
  slot = take ? slot0 + ci : slot;
}

// f(std::integral_constant<int, kI>()), ..., for kI < kN: a loop whose index
// is a constant expression (immediates, compile-time dispatch).
template <int kI, int kN, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (kI < kN) {
    f(std::integral_constant<int, kI>());
    static_for<kI + 1, kN>(f);
  }
}

// fold_tree<true> cut into eight pieces of four to six VALU instructions,
// for a kernel that places one piece after each of its MFMAs itself (the
// scheduler cannot spread the opaque scan blocks): pieces 0 and 1 the max3
// tree, 2 to 6 the reverse scan, 7 the update.  Same operations, same
// results.  Piece 1 completes the tree, so every score has been read by a
// compiler-visible instruction before the scan's asm reads it.
struct FoldPieces {
  float m0, m1, m2, m3, cm;
  int ci;
};

template <int kP, bool kRowSlots = false>
__device__ __forceinline__ void fold_piece(FoldPieces& f, const float (&s)[16], int slot0,
                                           float& mx, int& slot) {
  static_assert(kP >= 0 && kP < 8, "eight pieces");
  if constexpr (kP == 0) {
    f.m0 = max3_ieee(s[0], s[1], s[2]);
    f.m1 = max3_ieee(s[3], s[4], s[5]);
    f.m2 = max3_ieee(s[6], s[7], s[8]);
    f.m3 = max3_ieee(s[9], s[10], s[11]);
  } else if constexpr (kP == 1) {
    const float m4 = max3_ieee(s[12], s[13], s[14]);
    const float m5 = max3_ieee(s[15], f.m0, f.m1);
    const float m6 = max3_ieee(f.m2, f.m3, m4);
    f.cm = max3_ieee(m5, m6, -INFINITY);
    f.ci = reg_slot<kRowSlots>(15);
  } else if constexpr (kP == 2) {
    first_equal_regs<kRowSlots, 14>(f.ci, s, f.cm);
  } else if constexpr (kP == 3) {
    first_equal_regs<kRowSlots, 11>(f.ci, s, f.cm);
  } else if constexpr (kP == 4) {
    first_equal_regs<kRowSlots, 8>(f.ci, s, f.cm);
  } else if constexpr (kP == 5) {
    first_equal_regs<kRowSlots, 5>(f.ci, s, f.cm);
  } else if constexpr (kP == 6) {
    first_equal_regs<kRowSlots, 2>(f.ci, s, f.cm);
  } else {
    const bool take = f.cm > mx;
    mx = take ? f.cm : mx;
    slot = take ? slot0 + f.ci : slot;
  }
}

// fold_tree8: the same update over one half of the registers, 0..7 (rows
// 0..15 of the chunk) or 8..15 (rows 16..31), when the two halves of a chunk
// belong to different documents.  slot = slot0 + register index within the
// half (kRowSlots: its row offset, acc_row(8 + r, 0) = 16 + acc_row(r, 0)).
template <bool kUpper, bool kRowSlots = false>
__device__ __forceinline__ void fold_tree8(const float (&s)[16], int slot0, float& mx, int& slot) {
  constexpr int o = kUpper ? 8 : 0;
  // (reg_slot of the half's own index: slot0 carries the rest)
  const float m0 = max3_ieee(s[o + 0], s[o + 1], s[o + 2]);
  const float m1 = max3_ieee(s[o + 3], s[o + 4], s[o + 5]);
  const float m2 = max3_ieee(s[o + 6], s[o + 7], m0);
  const float cm = max3_ieee(m1, m2, -INFINITY);
  int ci = reg_slot<kRowSlots>(7);
#pragma unroll
  for (int r = 6; r >= 0; --r) ci = (s[o + r] == cm) ? reg_slot<kRowSlots>(r) : ci;
  const bool take = cm > mx;
  mx = take ? cm : mx;
  slot = take ? slot0 + ci : slot;
}

// fold_tree8 (row slots) cut into four pieces for a kernel that pins them
// beside its MFMAs: 0 the max3 tree, 1 and 2 the scan of registers 6..1,
// 3 registers 2..0 and the update.  Piece 3 repeats registers 2 and 1 to
// keep three compares per block (no wait-state padding); a descending
// re-scan ends on the same lowest register, so the result is fold_tree8's.
struct FoldPieces8 {
  float cm;
  int ci;
};

template <int kP, bool kUpper>
__device__ __forceinline__ void fold_piece8(FoldPieces8& f, const float (&s)[16], int slot0,
                                            float& mx, int& slot) {
  static_assert(kP >= 0 && kP < 4, "four pieces");
  constexpr int o = kUpper ? 8 : 0;
  if constexpr (kP == 0) {
    const float m0 = max3_ieee(s[o + 0], s[o + 1], s[o + 2]);
    const float m1 = max3_ieee(s[o + 3], s[o + 4], s[o + 5]);
    const float m2 = max3_ieee(s[o + 6], s[o + 7], m0);
    f.cm = max3_ieee(m1, m2, -INFINITY);
    f.ci = reg_slot<true>(7);
  } else if constexpr (kP == 1) {
    first_equal3<reg_slot<true>(6), reg_slot<true>(5), reg_slot<true>(4)>(f.ci, s[o + 6], s[o + 5],
                                                                            s[o + 4], f.cm);
  } else if constexpr (kP == 2) {
    first_equal3<reg_slot<true>(3), reg_slot<true>(2), reg_slot<true>(1)>(f.ci, s[o + 3], s[o + 2],
                                                                            s[o + 1], f.cm);
  } else {
    first_equal3<reg_slot<true>(2), reg_slot<true>(1), reg_slot<true>(0)>(f.ci, s[o + 2], s[o + 1],
                                                                            s[o + 0], f.cm);
    const bool take = f.cm > mx;
    mx = take ? f.cm : mx;
    slot = take ? slot0 + f.ci : slot;
  }
}

// The running maximum alone, for scans that write no argmax tape: fold_tree's
// max3 tree with the running max as its root's third input, so mx ends on
// the value fold_tree's strictly-greater update gives (the two can differ
// only in the sign of a zero maximum: the tree orders -0 below +0, the
// update keeps the earlier of equal values).  Cut into eight pieces of one
// v_max3 (one node of the tree each, piece 7 the root) for kernels that pin
// them beside their MFMAs; fold_max runs all eight.
struct MaxPieces {
  float n0, n1, n2, n3, n4, n5, n6;
};

template <int kP>
__device__ __forceinline__ void fold_max_piece(MaxPieces& f, const float (&s)[16], float& mx) {
  static_assert(kP >= 0 && kP < 8, "eight pieces");
  if constexpr (kP == 0) f.n0 = max3_ieee(s[0], s[1], s[2]);
  else if constexpr (kP == 1) f.n1 = max3_ieee(s[3], s[4], s[5]);
  else if constexpr (kP == 2) f.n2 = max3_ieee(s[6], s[7], s[8]);
  else if constexpr (kP == 3) f.n3 = max3_ieee(s[9], s[10], s[11]);
  else if constexpr (kP == 4) f.n4 = max3_ieee(s[12], s[13], s[14]);
  else if constexpr (kP == 5) f.n5 = max3_ieee(s[15], f.n0, f.n1);
  else if constexpr (kP == 6) f.n6 = max3_ieee(f.n2, f.n3, f.n4);
  else mx = max3_ieee(f.n5, f.n6, mx);
}

__device__ __forceinline__ void fold_max(const float (&s)[16], float& mx) {
  MaxPieces f;
  static_for<0, 8>([&](auto p) { fold_max_piece<decltype(p)::value>(f, s, mx); });
}

// The same over one half of the registers (fold_tree8's rows), four pieces.
struct MaxPieces8 {
  float n0, n1, n2;
};

template <int kP, bool kUpper>
__device__ __forceinline__ void fold_max_piece8(MaxPieces8& f, const float (&s)[16], float& mx) {
  static_assert(kP >= 0 && kP < 4, "four pieces");
  constexpr int o = kUpper ? 8 : 0;
  if constexpr (kP == 0) f.n0 = max3_ieee(s[o + 0], s[o + 1], s[o + 2]);
  else if constexpr (kP == 1) f.n1 = max3_ieee(s[o + 3], s[o + 4], s[o + 5]);
  else if constexpr (kP == 2) f.n2 = max3_ieee(s[o + 6], s[o + 7], f.n0);
  else mx = max3_ieee(f.n1, f.n2, mx);
}

template <bool kUpper>
__device__ __forceinline__ void fold_max8(const float (&s)[16], float& mx) {
  MaxPieces8 f;
  static_for<0, 4>([&](auto p) { fold_max_piece8<decltype(p)::value, kUpper>(f, s, mx); });
}

// The maxima of the two wave halves merged in every lane (for folds that
// never take a NaN): both halves' values from one v_permlane32_swap.
__device__ __forceinline__ float merge_halves_max(float mx) {
  const auto ms = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, mx),
                                                   __builtin_bit_cast(uint32_t, mx), false, false);
  return __builtin_fmaximum_numf(__builtin_bit_cast(float, (uint32_t)ms[0]),
                                 __builtin_bit_cast(float, (uint32_t)ms[1]));
}

// running_max_seq: the sequential scan itself, with row masking, for the
// HBM-bound scans (fewest live registers).  `rowbits` is the
// chunk validity shifted to this lane half (bit 8*(r/4) + r%4 = register r);
// kMasked = false skips the test for fully valid chunks.  The register index
// r is a chunk-local immediate folded into `slot` once per chunk: three VALU
// ops per score.
template <bool kMasked>
__device__ __forceinline__ void running_max_seq(const float (&s)[16], uint32_t rowbits,
                                                int slot0, float& mx, int& slot) {
  int rc = -1;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const bool ok = !kMasked || ((rowbits >> (8 * (r >> 2) + (r & 3))) & 1u);
    const bool take = ok && s[r] > mx;
    mx = take ? s[r] : mx;
    rc = take ? r : rc;
  }
  slot = rc >= 0 ? slot0 + rc : slot;
}

// 1-based document token of a slot for a lane in half h; 0 = none.
__device__ __forceinline__ int slot_to_token(int slot, int h) {
  return slot < 0 ? 0 : (slot >> 4) * kTile + acc_row(slot & 15, h) + 1;
}

// The same for a stream of 16-row units: slot = (v + 1) * 16 + r, where the
// chunk's row 0 is document row 16 v (v = -1 when the document starts in the
// chunk's second half, whose registers are 8..15).
// (masked with the sign of the slot, not selected: no control flow inside
// a fold that the scheduler interleaves with MFMAs)
__device__ __forceinline__ int slot_to_token16(int slot, int h) {
  const int t = ((slot >> 4) - 1) * 16 + acc_row(slot & 15, h) + 1;
  return t & ~(slot >> 31);
}

// Cross-lane exchanges without LDS.  v_permlane32_swap(a, b) trades lanes
// 32-63 of `a` with lanes 0-31 of `b` and returns both; with a = b = x that
// gives {[x_lo, x_lo], [x_hi, x_hi]}, so lane l finds x[l ^ 32] in the
// second result when it is in the low half (h = 0) and in the first when it
// is in the high half.  (ds_bpermute, behind __shfl_xor, costs an LDS round
// trip per step of a reduction.)
__device__ __forceinline__ uint32_t lane_xor32(uint32_t x, int h) {
  const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return h ? r[0] : r[1];
}

// v + v[lane dpp-permuted] for a DPP control (quad_perm / row_ror).
template <int kCtrl>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                           0, __builtin_bit_cast(int, v), kCtrl, 0xf, 0xf, false));
}

// NaN test on the bit pattern (no floating-point compare for the compiler
// to rewrite).
__device__ __forceinline__ bool is_nan_bits(float x) {
  return (__builtin_bit_cast(uint32_t, x) & 0x7fffffffu) > 0x7f800000u;
}

// Merge the (max, token) of lanes l and l^32, which hold disjoint document
// rows of the same query token.  Equal maxima keep the lower token, matching
// a sequential ascending scan.  h = lane / 32.
__device__ __forceinline__ void merge_halves(float& mx, int& tok, int h) {
  const float omx = __builtin_bit_cast(float, lane_xor32(__builtin_bit_cast(uint32_t, mx), h));
  const int otok = (int)lane_xor32((uint32_t)tok, h);
  // Bitwise, not short-circuit: no exec-mask branches.  A NaN maximum can
  // only be the first valid token's (take_first_row) and it stands.
  const bool nan_here = is_nan_bits(mx), nan_there = is_nan_bits(omx);
  const bool take = (otok != 0) & !nan_here &
                    ((tok == 0) | nan_there | (omx > mx) | ((omx == mx) & (otok < tok)));
  mx = take ? omx : mx;
  tok = take ? otok : tok;
}

// The (max, token) of the two wave halves merged in every lane, for folds
// that never take a NaN (merge_halves<true>'s rule): one v_permlane32_swap
// of each value gives every lane the low half's value in its first result
// and the high half's in its second, so every lane merges (low, high) in the
// same order and no lane needs its own half picked out.
__device__ __forceinline__ void merge_halves_all(float& mx, int& tok) {
  const auto ms = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, mx),
                                                   __builtin_bit_cast(uint32_t, mx), false, false);
  const auto ts = __builtin_amdgcn_permlane32_swap((uint32_t)tok, (uint32_t)tok, false, false);
  mx = __builtin_bit_cast(float, (uint32_t)ms[0]);
  tok = (int)ts[0];
  const float omx = __builtin_bit_cast(float, (uint32_t)ms[1]);
  const int otok = (int)ts[1];
  // (tokens <= 0 mean none)
  const bool take = (otok > 0) & ((tok <= 0) | (omx > mx) | ((omx == mx) & (otok < tok)));
  mx = take ? omx : mx;
  tok = take ? otok : tok;
}

// The reference's running max starts empty, `arg == 0 || s > mx`
// (kernels_forward.jl:49-52, forward_pair.jl:82-85): the first valid
// document token u0 is taken whatever its score, and only a strictly greater
// score replaces it.  So a NaN score at u0 sticks (nothing compares greater
// than NaN), all-(-Inf) scores keep u0, and NaN scores after u0 are skipped.
// take_first_row starts the running max of the lanes holding u0 on u0's
// score, in the first chunk with a valid row -- recognised without extra
// state: no lane has taken a row yet.  The regular fold then continues with
// strictly-greater takes (u0 itself is not greater than itself), and
// merge_halves lets a NaN win, which only u0 can hold.  For finite scores
// this gives exactly the plain max with first-index ties.  Uniform control.
__device__ __forceinline__ void take_first_row(const float (&s)[16], uint32_t m32, int h, int ch,
                                               float& mx, int& slot) {
  if (m32 != 0u && __ballot(slot >= 0) == 0ull) {
    const int row = __builtin_ctz(m32);
    const int reg = ((row >> 3) << 2) | (row & 3);  // acc_row(reg, (row >> 2) & 1) == row
    f32x16 sv;  // a uniform index into a register vector: one v_movrels
#pragma unroll
    for (int r = 0; r < 16; ++r) sv[r] = s[r];
    const float v = sv[reg];
    const bool mine = h == ((row >> 2) & 1);
    mx = mine ? v : mx;
    slot = mine ? ch * 16 + reg : slot;
  }
}

// Sum over lanes 0-31, returned in every lane (wave-uniform).  After
// merge_halves both wave halves hold the same 32 per-token partials, so this
// is the score.  Quad butterflies and row rotations by DPP leave each row
// of 16 lanes holding its sum; rows 0 and 1 are then read with v_readlane.
// (v_permlane16_swap would do the last step in vector registers, but this
// compiler folds `r[0] + r[1]` of its two results into `r[0] + r[0]`.)
__device__ __forceinline__ float row_sums(float v) {
  v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
  v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
  v = dpp_add<0x124>(v);  // row_ror:4
  v = dpp_add<0x128>(v);  // row_ror:8 -> each row of 16 holds its sum
  return v;
}
__device__ __forceinline__ float half_sum(float v) {
  const int bits = __builtin_bit_cast(int, row_sums(v));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 0)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 16));
}

// half_sum left in lanes 16-31 (and 48-63) instead of read out: a
// row_bcast:15 DPP add puts row 0's sum into row 1 (row 2's into row 3),
// the same two row sums half_sum adds (row 1's + row 0's).
__device__ __forceinline__ float half_sum_in_lanes(float v) {
  v = row_sums(v);
  return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                           0, __builtin_bit_cast(int, v), 0x142, 0xa, 0xf, false));
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

}  // namespace fms
