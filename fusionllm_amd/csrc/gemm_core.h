// gemm_core.h — building blocks of the gfx950 bf16 GEMM main loop shared by the
// grouped expert products.
//
// Tile: 256 x 256 outputs per 512-thread workgroup (8 waves, 4 x 2, each wave a
// 64 x 128 sub-tile of 4 x 8 blocks of v_mfma_f32_16x16x32_bf16), K stepped by
// 64 through two LDS stages of 64 KB (operand rows of 128 bytes, K-contiguous).
//
// * Global -> LDS copies use global_load_lds_dwordx4 (16 bytes per lane written
//   straight into LDS, no VGPR round trip).  One wave instruction writes 1 KB
//   of LDS = 8 rows; the 16-byte chunks of a row are XOR-swizzled
//   (slot = chunk ^ (row & 7), swzk below) by choosing which global chunk a
//   lane fetches, which makes the fragment reads below free of bank conflicts.
// * The copies and the LDS fragment reads are issued from inline assembly so
//   that the compiler neither reorders them nor inserts conservative
//   vmcnt(0) waits between the copies and the reads; every wait is explicit.
// * 32-deep K steps are split into four blocks of 8 MFMAs.  Each block reads,
//   interleaved with its MFMAs, the fragments that the same block of the next
//   step needs: the eight B-side fragments ("P") are reloaded in place right
//   after their last use, the four A-side fragments ("Q") are double buffered.
// * MFMA operands are swapped (srcA = B fragment, srcB = A fragment), so that a
//   lane's 4 accumulators hold 4 consecutive output columns of one row:
//   acc[i][j] of lane l = C[16 i + l % 16][16 j + 4 (l / 16) + 0..3].
#pragma once

#include "fmoe_common.h"

namespace fmoe {
namespace core {

constexpr int BM = 256, BN = 256, BK = 64, NT = 512;
constexpr int RB = BK * 2;                  // LDS bytes per operand row
constexpr int A_BYTES = BM * RB;            // 32 KB
constexpr int STAGE = (BM + BN) * RB;       // 64 KB
constexpr int EPI = 4096;                   // epilogue staging bytes per wave
constexpr int SMEM = 2 * STAGE + 8 * EPI;   // 160 KB: the whole LDS of a CU
constexpr int WM = 4, WN = 2;               // wave grid
constexpr int WTM = BM / WM, WTN = BN / WN; // 64 x 128 per wave
constexpr int FM = WTM / 16, FN = WTN / 16; // 4 x 8 blocks of 16 x 16
constexpr int LA = 4, LB = 4, LT = LA + LB; // copy instructions per lane per stage

// Operand stages: 16-byte chunk c of 128-byte row r sits at slot c ^ swzk(r).
// With this swizzle the fragment reads below (lane l: row l % 16 of a
// 16-row group, chunk l / 16 [+4]) are free of LDS bank conflicts on gfx950
// (measured with SQ_LDS_BANK_CONFLICT; folding bit 3 of the row into the
// swizzle gave 2-way conflicts).
__device__ __forceinline__ int swzk(int r) { return r & 7; }
// Epilogue staging of 128-byte rows: slot c ^ swz(r).
__device__ __forceinline__ int swz(int r) { return (r ^ (r >> 3)) & 7; }

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  // generic -> LDS address space (a C-style cast is the only form clang accepts)
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) uint8_t*)p));
}

// One 16-byte-per-lane copy global -> LDS.  lds: wave-uniform LDS byte address
// of the 1 KB the wave writes; base: wave-uniform global address; voff: this
// lane's byte offset from base.
__device__ __forceinline__ void copy16(uint32_t lds, const void* base, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2\n" ::"s"(lds), "v"(voff), "s"(base)
               : "memory");
}

// Scalar load of two consecutive ints at a wave-uniform address.  The compiler
// turns uniform reads issued after the copies (inline assembly that clobbers
// memory) into vector loads whose vmcnt wait would also wait for every copy in
// flight; a scalar load is tracked by lgkmcnt instead.
__device__ __forceinline__ int2 sload2(const int32_t* p) {
  int2 v;
  asm volatile("s_load_dwordx2 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)\n" : "=s"(v) : "s"(p) : "memory");
  return v;
}

// Scalar load of eight consecutive ints at a wave-uniform address (tracked by
// lgkmcnt, waited for at once, as sload2).
typedef int i32x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ i32x8 sload8(const int32_t* p) {
  i32x8 v;
  asm volatile("s_load_dwordx8 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)\n" : "=s"(v) : "s"(p) : "memory");
  return v;
}

// One 4-byte-per-lane copy global -> LDS (lane l writes LDS bytes lds + 4 l).
__device__ __forceinline__ void copy4(uint32_t lds, const void* base, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2\n" ::"s"(lds), "v"(voff), "s"(base) : "memory");
}

// Wait until at most N vector-memory operations of this wave are in flight and
// its LDS reads are done, then synchronise the workgroup.
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier\n" ::"n"(N) : "memory");
}

#define FMOE_MF(c, a, b) "v_mfma_f32_16x16x32_bf16 " c ", " a ", " b ", " c "\n"
#define FMOE_DS(d, p) "ds_read_b128 " d ", " p "\n"

// Block x of a 32-deep K step: acc[q][2x + p] += A_q (x) B_(2x+p) for q = 0..3,
// p = 0..1.  Reads next-step fragments: Q'[x] (A side) into nq, and P[2x],
// P[2x+1] (B side) in place after their last use.  WAIT = lgkmcnt bound that
// guarantees the fragments this block consumes have arrived.
// The reads are still in flight when the statement ends: their destinations
// are read-write operands ("+v"), so each keeps one register across the loop
// that is consumed only by a later block8, after the s_waitcnt that covers
// it (tests/test_host.py checks the built code for any other access to a
// pending ds_read destination).
template <int WAIT>
__device__ __forceinline__ void block8(f32x4& c00, f32x4& c01, f32x4& c02, f32x4& c03, f32x4& c10, f32x4& c11,
                                       f32x4& c12, f32x4& c13, bf16x8& p0, bf16x8& p1, const bf16x8& q0,
                                       const bf16x8& q1, const bf16x8& q2, const bf16x8& q3, bf16x8& nq,
                                       uint32_t aq, uint32_t ap0, uint32_t ap1) {
  asm volatile(
      "s_waitcnt lgkmcnt(%[wt])\n"
      FMOE_DS("%[nq]", "%[aq]")
      FMOE_MF("%[c00]", "%[p0]", "%[q0]") FMOE_MF("%[c01]", "%[p0]", "%[q1]")
      FMOE_MF("%[c02]", "%[p0]", "%[q2]") FMOE_MF("%[c03]", "%[p0]", "%[q3]")
      FMOE_DS("%[p0]", "%[ap0]")
      FMOE_MF("%[c10]", "%[p1]", "%[q0]") FMOE_MF("%[c11]", "%[p1]", "%[q1]")
      FMOE_MF("%[c12]", "%[p1]", "%[q2]") FMOE_MF("%[c13]", "%[p1]", "%[q3]")
      FMOE_DS("%[p1]", "%[ap1]")
      : [c00] "+v"(c00), [c01] "+v"(c01), [c02] "+v"(c02), [c03] "+v"(c03), [c10] "+v"(c10), [c11] "+v"(c11),
        [c12] "+v"(c12), [c13] "+v"(c13), [p0] "+v"(p0), [p1] "+v"(p1), [nq] "+v"(nq)
      : [q0] "v"(q0), [q1] "v"(q1), [q2] "v"(q2), [q3] "v"(q3), [aq] "v"(aq), [ap0] "v"(ap0), [ap1] "v"(ap1),
        [wt] "n"(WAIT));
}

#undef FMOE_MF
#undef FMOE_DS

// LDS address of fragment f of one operand: the lane's row (16 f + l % 16 of
// the wave's block) at chunk (l / 16 + 4 * step half), swizzled.  For rows
// r = base + 16 f + l % 16 with base % 16 == 0, swzk(r) = l & 7, so every
// fragment address is x + 2048 f for one per-lane x (the wave's row block and
// l's swizzle), and the K half is one XOR of 64 (chunk bit 2).
__device__ __forceinline__ uint32_t frag_base(int row0, int lane) {
  const int t = (lane >> 4) ^ (lane & 7);
  return static_cast<uint32_t>((row0 + (lane & 15)) * RB + (t << 4));
}
template <int F, int KX>
__device__ __forceinline__ uint32_t frag_addr(uint32_t x, uint32_t src) {
  return (x ^ static_cast<uint32_t>(KX)) + (src + 2048u * F);
}

// One 32-deep K step of the wave's 64 x 128 sub-tile on fragments P (B side,
// 8) and Qc (A side, 4), reading the next step's fragments (Qn, P in place)
// from the stage at LDS address src, K half KX (0 or 64).  xa / xb: frag_base
// of the wave's A rows and B rows (B rows offset by A_BYTES in src).
template <int KX>
__device__ __forceinline__ void kstep(f32x4 (&acc)[FM][FN], bf16x8 (&P)[FN], bf16x8 (&Qc)[4], bf16x8 (&Qn)[4],
                                      uint32_t xa, uint32_t xb, uint32_t src) {
  const uint32_t srcb = src + A_BYTES;
  // Block 0 needs Q'[3] of the previous step (two reads younger): lgkmcnt(2);
  // block x > 0 needs P[2x], P[2x+1] of the previous step (nine reads younger).
  block8<2>(acc[0][0], acc[1][0], acc[2][0], acc[3][0], acc[0][1], acc[1][1], acc[2][1], acc[3][1], P[0], P[1],
            Qc[0], Qc[1], Qc[2], Qc[3], Qn[0], frag_addr<0, KX>(xa, src), frag_addr<0, KX>(xb, srcb),
            frag_addr<1, KX>(xb, srcb));
  block8<9>(acc[0][2], acc[1][2], acc[2][2], acc[3][2], acc[0][3], acc[1][3], acc[2][3], acc[3][3], P[2], P[3],
            Qc[0], Qc[1], Qc[2], Qc[3], Qn[1], frag_addr<1, KX>(xa, src), frag_addr<2, KX>(xb, srcb),
            frag_addr<3, KX>(xb, srcb));
  block8<9>(acc[0][4], acc[1][4], acc[2][4], acc[3][4], acc[0][5], acc[1][5], acc[2][5], acc[3][5], P[4], P[5],
            Qc[0], Qc[1], Qc[2], Qc[3], Qn[2], frag_addr<2, KX>(xa, src), frag_addr<4, KX>(xb, srcb),
            frag_addr<5, KX>(xb, srcb));
  block8<9>(acc[0][6], acc[1][6], acc[2][6], acc[3][6], acc[0][7], acc[1][7], acc[2][7], acc[3][7], P[6], P[7],
            Qc[0], Qc[1], Qc[2], Qc[3], Qn[3], frag_addr<3, KX>(xa, src), frag_addr<6, KX>(xb, srcb),
            frag_addr<7, KX>(xb, srcb));
}

// ---- weights read as they lie ([K, N] row-major, N contiguous): the backward
// dX products (dh = d_out * w2, dx = [da | db] * [w1; w3]) take their B
// operand from the nn.Linear weights without a transposed copy.
// B stage: 64 k rows of 512 bytes (256 n values), copied as they lie; the
// 32-byte windows of a k row are XOR-swizzled by wsw(k row), and fragments
// are read with ds_read_b64_tr_b16, which returns to lane (h = l / 16,
// i = l % 16) column i of the 4 x 4 block of 16-bit values that the
// group's source lanes 4 j + q address (row j, 4 values at column 4 q); two
// such reads, 4 k rows apart, give a lane 8 consecutive k of one n.  A
// 64-bit read cannot name half of an inline-assembly operand, so in this
// variant all LDS reads are compiler loads (the compiler places the waits
// for them) and only the MFMA groups are inline assembly.
__device__ __forceinline__ int wsw(int r) { return (r & 3) | (((r >> 3) & 1) << 2); }

// Lane's address of B fragment 0 (K half 0) within a stage, relative to the
// stage base: k row 8 h + jq (+4 for the second read), window (8 wn + fr) for
// the wave's 128 columns, fr = wsw(8 h + jq).  Fragment f: ^ (f << 5); the
// second 32-deep half of the stage: + 32 rows.
__device__ __forceinline__ uint32_t trb_base(int wn, int lane) {
  const int h = lane >> 4, jq = (lane >> 2) & 3, q = lane & 3;
  const int fr = jq | ((h & 1) << 2);
  return static_cast<uint32_t>(A_BYTES + (8 * h + jq) * 512 + ((8 * wn + fr) << 5) + 8 * q);
}
constexpr uint32_t TRB_KHALF = 32 * 512;

typedef short s16x4 __attribute__((ext_vector_type(4)));
// One B fragment: 8 consecutive k of the lane's n (two transposing reads).
__device__ __forceinline__ bf16x8 trb_frag(uint32_t addr) {
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uintptr_t)addr);
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uintptr_t)(addr + 2048u));
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

#define FMOE_MFA(c, a, b) "v_mfma_f32_16x16x32_bf16 " c ", " a ", " b ", " c "\n"
// Four MFMAs of one B fragment: acc[0..3][j] += P[j] (x) Q[0..3].  The LDS
// reads of this variant are compiler loads, so the compiler places exact
// waits for them before the statement that consumes them.
__device__ __forceinline__ void block4m(f32x4& c0, f32x4& c1, f32x4& c2, f32x4& c3, const bf16x8& p,
                                        const bf16x8& q0, const bf16x8& q1, const bf16x8& q2, const bf16x8& q3) {
  asm volatile(FMOE_MFA("%[c0]", "%[p]", "%[q0]") FMOE_MFA("%[c1]", "%[p]", "%[q1]")
               FMOE_MFA("%[c2]", "%[p]", "%[q2]") FMOE_MFA("%[c3]", "%[p]", "%[q3]")
               : [c0] "+v"(c0), [c1] "+v"(c1), [c2] "+v"(c2), [c3] "+v"(c3)
               : [p] "v"(p), [q0] "v"(q0), [q1] "v"(q1), [q2] "v"(q2), [q3] "v"(q3)
               : "memory");
}
#undef FMOE_MFA

// kstep with B read as it lies.  Block x: MFMAs with P[2x], then the next
// step's Q'[x] (A side, double buffered) and P[2x] (in place), MFMAs with
// P[2x+1], then P[2x+1].  KH: the next fragments come from the second (1) or
// first (0) 32-deep half of the stage at src.  (Measured against the
// transposed-copy path on MI355X, outputs bit-identical: the two dX products
// 1 % slower at C2 and 2 % at C5, less than the transposed copies cost.)
template <int KH>
__device__ __forceinline__ void kstep_t(f32x4 (&acc)[FM][FN], bf16x8 (&P)[FN], bf16x8 (&Qc)[4], bf16x8 (&Qn)[4],
                                        uint32_t xa, uint32_t xbt, uint32_t src) {
  constexpr int KX = KH ? 64 : 0;
  const uint32_t bb = src + (KH ? TRB_KHALF : 0u);
  typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;
#define FMOE_BLK(X)                                                                                              \
  block4m(acc[0][2 * X], acc[1][2 * X], acc[2][2 * X], acc[3][2 * X], P[2 * X], Qc[0], Qc[1], Qc[2], Qc[3]);        \
  Qn[X] = *(const lds_bf16x8*)(uintptr_t)frag_addr<X, KX>(xa, src);                                                \
  P[2 * X] = trb_frag(bb + (xbt ^ ((2u * X) << 5)));                                                              \
  block4m(acc[0][2 * X + 1], acc[1][2 * X + 1], acc[2][2 * X + 1], acc[3][2 * X + 1], P[2 * X + 1], Qc[0], Qc[1],  \
          Qc[2], Qc[3]);                                                                                          \
  P[2 * X + 1] = trb_frag(bb + (xbt ^ ((2u * X + 1) << 5)));
  FMOE_BLK(0)
  FMOE_BLK(1)
  FMOE_BLK(2)
  FMOE_BLK(3)
#undef FMOE_BLK
}

}  // namespace core
}  // namespace fmoe
