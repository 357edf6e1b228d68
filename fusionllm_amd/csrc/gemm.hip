// gemm.hip — grouped bf16 GEMMs on CDNA4 matrix cores
// (v_mfma_f32_16x16x32_bf16) for the expert SwiGLU products of FusionLLM's
// DeepSeekMoE.
//
// Replaces SwiGLUExpert.forward (models/moe.py:20-21) called once per active
// expert in the loop of moe.py:66-76 and once for the shared expert
// (moe.py:86), and the autograd of those calls.  All experts (and the shared
// expert as one more group) go into a single launch per product; the tile ->
// (expert, rows) mapping is computed on the device from offsets[], so no
// host synchronisation is needed for the ragged, skewed expert sizes.
//
// Row-grouped products (rows_gemm_kernel, modes below): persistent
// workgroups of 8 waves walk 256 x 256 output tiles in an XCD-contiguous
// order.  Both operands are K-contiguous in memory and reach LDS through
// global_load_lds copies (no registers) into a two-stage ring of 64-deep K
// steps that runs on across tile boundaries; a wave owns a 64 x 128 block
// and runs the hand-scheduled K step of gemm_core.h.  The epilogue stages
// each 16-row slice through LDS for 16-byte stores and fuses the SwiGLU
// (forward: a | b and h = silu(a) * b; backward: da, db from dh, a, b).  The
// tiles of the last, partial round of the plain-output products are split
// along K, with fp32 partials summed in range order by split_reduce_kernel.
//
// Weight gradients (wgrad_tr_kernel): work units (group, K chunk, tile);
// both operands are MN-contiguous, copied as they lie and read with
// ds_read_b64_tr_b16 (transposing LDS reads); multi-chunk groups write fp32
// partials that wgrad_reduce_kernel adds in chunk order.
//
// Decode-sized launches send groups of at most kSmallM rows to
// small_gemm_kernel, which streams the weights once (when no group of the
// launch can exceed 2 kSmallM rows, every group, in slabs of kSmallM).
#include <atomic>

#include "fmoe_common.h"
#include "gemm_core.h"

namespace fmoe {

// ---- row-grouped products ---------------------------------------------------
// The activations are row-major [rows, K] (K-contiguous).  The weights are
// the nn.Linear weights as they lie: [out, in] with K = in for the forward
// products (K-contiguous, read like the activations), and [K, N] row-major
// for the backward dX products (dh = d_out * w2 reads w2 [dim, inter];
// dx = [da | db] * [w1; w3] reads w1, w3 [inter, dim]), whose B stages are
// copied as they lie and read with transposing LDS reads (gemm_core.h).
enum GemmMode { GATEUP_FWD = 0, DOWN_FWD = 1, DOWN_BWD = 2, GATEUP_BWD = 3 };

struct GemmArgs {
  const uint16_t* a_routed;  // [rows_routed, K], or with gather: x [T, K]
  const int32_t* gather;     // GATEUP_FWD tiled kernel: routed row r reads a_routed row gather[r] / gather_k
                             // (nullptr: row r; launches of more than kSmallLaunchRows rows only)
  int gather_k;
  uint64_t gather_magic;     // slot_div_magic(gather_k)
  const uint16_t* a_shared;  // [rows_shared, K] (nullptr: rows follow the routed rows)
  int64_t lda;
  const int32_t* offsets;  // [E+1], device
  int E;
  int rows_routed;
  int rows_shared;
  int K;        // reduction length
  int N;        // output columns (GATEUP_FWD: inter = h columns)
  int inter;    // SwiGLU width (GATEUP_FWD, DOWN_BWD)
  int64_t ldb;  // leading dimension of the weight operand (row length as it lies in memory)
  uint16_t* c0;  // main output (ab / out / d_ab / dx_rows)
  uint16_t* c1;  // GATEUP_FWD: h
  const uint16_t* aux;  // DOWN_BWD: ab
  int64_t ldc0, ldc1, ldaux;
  const uint16_t* b0[FMOE_MAX_EXPERTS + 1];  // w1 (GATEUP_*) / w2 (DOWN_*)
  const uint16_t* b1[FMOE_MAX_EXPERTS + 1];  // w3 (GATEUP_*)
  int small_max;  // groups with 1 .. small_max rows go to small_gemm_kernel (0: none)
  int small_compact;  // DOWN_FWD small kernel: the grid covers only groups with rows
  float* split_ws;  // fp32 partials of the K-split tiles of the last round (nullptr: no split)
};

// ---- tiled row-grouped kernel ----------------------------------------------
// Persistent: a grid of at most one workgroup per CU walks the tiles
// t = blockIdx.x, blockIdx.x + gridDim.x, ...  Tiles are enumerated group by
// group (experts 0..E-1, then the shared expert), m tile major; the tile ->
// (group, rows) map comes from offsets[] on the device.  The global -> LDS
// copies run as one continuous two-stage ring over all K steps of all of a
// workgroup's tiles, so the next tile's first operands arrive while the current
// tile finishes and writes its epilogue.  Rows past a group's end and weight
// rows past N are clamped to the last valid one (their products are never
// stored), so no operand is read out of bounds.

// Tile t -> (group g, m tile tm, n tile tn, first row, group rows); false if t
// is past the last tile.
// offsets: args.offsets passed as a separate restrict pointer, so that these
// uniform reads become scalar loads (a vector load would need a vmcnt wait that
// also waits for the in-flight operand copies).
__device__ __forceinline__ bool locate_tile(const GemmArgs& a, const int32_t* __restrict__ offsets, int tiles_n,
                                            int t, int& g, int& tm, int& tn, int& row_base, int& M) {
  const int G = a.E + (a.rows_shared > 0 ? 1 : 0);
  for (g = 0; g < G; ++g) {
    if (g < a.E) {
      const int2 o = core::sload2(offsets + g);
      row_base = o.x;
      M = o.y - o.x;
    } else {
      row_base = a.rows_routed;
      M = a.rows_shared;
    }
    const int nt = (M <= a.small_max) ? 0 : ((M + core::BM - 1) / core::BM) * tiles_n;
    if (t < nt) {
      tm = t / tiles_n;
      tn = t - tm * tiles_n;
      return true;
    }
    t -= nt;
  }
  return false;
}

__device__ __forceinline__ int count_tiles(const GemmArgs& a, const int32_t* __restrict__ offsets, int tiles_n) {
  const int G = a.E + (a.rows_shared > 0 ? 1 : 0);
  int total = 0;
  for (int g = 0; g < G; ++g) {
    int M = a.rows_shared;
    if (g < a.E) {
      const int2 o = core::sload2(offsets + g);
      M = o.y - o.x;
    }
    total += (M <= a.small_max) ? 0 : ((M + core::BM - 1) / core::BM) * tiles_n;
  }
  return total;
}

// Store instructions per lane in the epilogue of a full tile (they may still
// be in flight at the next barrier; see the wait there).
template <int MODE>
constexpr int epi_stores() {
  return MODE == GATEUP_FWD ? 24 : (MODE == DOWN_BWD ? 32 : 16);
}

// K-split of the last, partial round of tiles.  With T tiles on P
// workgroups, the T mod P tiles of the last round would run on a fraction of
// the CUs; instead each is split into S K ranges (S <= 4, R * S <= P, at
// least 4 K steps per range) whose fp32 partials a split reduction adds in
// range order before the product's epilogue.  Work items: tiles 0 .. full-1
// whole, then R * S ranges.
// Only for runs of fewer than kSplitMaxRounds full rounds.  Measured on
// MI355X (split minus whole, same process): at T=16384, d=768, I=2048 the
// split gains 12 us on the down product (2 rounds, 32 K steps), 47 us on the
// gate/up backward (2 rounds, 64 K steps) and 3 us on the down backward (6
// rounds, 12 K steps) but loses 9 us on the gate/up forward (12 rounds, 12
// K steps); at d=2048, I=1408, 64 experts (21 to 38 rounds) it loses 1 to
// 15 us on every product.  Over many rounds the workgroups' finishing times
// spread by about a tile anyway, and the partials' HBM traffic (written and
// read once, 256 KB per range) is then not repaid.
struct SplitPlan {
  int full, R, S;
  __device__ __forceinline__ int items() const { return full + R * S; }
};
constexpr int kSplitMaxS = 4;       // K ranges per split tile
constexpr int kSplitMaxRounds = 8;  // full rounds above which no tile is split
constexpr int kReduceParts = 16;  // blocks of a split reduction per split tile, 16 rows each

template <int MODE>
__device__ __forceinline__ SplitPlan split_plan(const GemmArgs& a, int T, int P, int nk) {
  SplitPlan sp{T, 0, 1};
  if (a.split_ws == nullptr || T <= 0) return sp;
  const int R = T % P;
  if (R == 0 || T / P >= kSplitMaxRounds) return sp;
  int S = min(P / R, kSplitMaxS);
  S = min(S, nk / 4);
  if (S < 2) return sp;
  sp.full = T - R;
  sp.R = R;
  sp.S = S;
  return sp;
}
// Workgroup b runs on XCD b % 8 (round-robin dispatch over the 8 XCDs of an
// MI355X, each with its own L2).  Item i of round r of workgroup b is
// r * P + xcd_slot(b): the workgroups of one XCD take a contiguous range of
// items, so the tiles that share operand rows (consecutive n tiles of one m
// tile) meet in the same L2.
__device__ __forceinline__ int xcd_slot(int b, int P) {
  return (P % 8 == 0) ? (b % 8) * (P / 8) + b / 8 : b;
}

// Work item -> tile, first K step, K steps, partial slot (-1: whole tile).
__device__ __forceinline__ void split_item(const SplitPlan& sp, int nk, int item, int& tile, int& k0, int& kn,
                                           int& slot) {
  if (item < sp.full) {
    tile = item;
    k0 = 0;
    kn = nk;
    slot = -1;
  } else {
    const int j = item - sp.full;
    const int s = j % sp.S;
    tile = sp.full + j / sp.S;
    k0 = s * nk / sp.S;
    kn = (s + 1) * nk / sp.S - k0;
    slot = j;
  }
}

// 16-byte global store / load; nt marks data streamed through once (the
// SwiGLU activations a|b and h, read again only in the backward pass, and
// their gradient), so it does not displace operands from the caches.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void store16(uint16_t* p, const uint4& v, bool nt) {
  if (nt) {
    const u32x4 q = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(q, reinterpret_cast<u32x4*>(p));
  } else {
    *reinterpret_cast<uint4*>(p) = v;
  }
}
__device__ __forceinline__ uint4 load16(const uint16_t* p, bool nt) {
  if (nt) {
    const u32x4 q = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(q.x, q.y, q.z, q.w);
  }
  return *reinterpret_cast<const uint4*>(p);
}

// SwiGLU backward of 8 columns (h = s * b, s = bf16(silu(a)); dh arrives
// bf16-rounded): da = bf16(bf16(dh * b) * silu'(a)), db = bf16(dh * s), with
// silu(a) = a * sg and silu'(a) = sg * (1 + a (1 - sg)) = sg + silu(a) (1 - sg).
__device__ __forceinline__ void swiglu_bwd8(const uint4& dhv, const uint4& av, const uint4& bv, uint4& dav,
                                            uint4& dbv) {
  float dh[8], af[8], bfv[8], da[8], db[8];
  unpack8(dhv, dh);
  unpack8(av, af);
  unpack8(bv, bfv);
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const float sg0 = fast_sigmoid(af[e]), sg1 = fast_sigmoid(af[e + 1]);
    const float sa0 = af[e] * sg0, sa1 = af[e + 1] * sg1;
    float sv0 = sa0, sv1 = sa1, ds0 = dh[e] * bfv[e], ds1 = dh[e + 1] * bfv[e + 1];
    bf_round2(sv0, sv1);
    bf_round2(ds0, ds1);
    da[e] = ds0 * fmaf(sa0, 1.0f - sg0, sg0);
    da[e + 1] = ds1 * fmaf(sa1, 1.0f - sg1, sg1);
    db[e] = dh[e] * sv0;
    db[e + 1] = dh[e + 1] * sv1;
  }
  dav = pack8(da);
  dbv = pack8(db);
}

// Down-backward epilogue of a full tile (this wave's 64 x 128 block of dh in
// acc).  The SwiGLU backward costs about as many instructions per element as
// the block has accumulators, so the block is first staged whole: dh rounded
// to bf16, through the wave's 4 KB of LDS one 16-row slice at a time, read
// back as 16-byte row segments (64 registers, the accumulators are then
// free).  The a|b loads then run as a pipeline two slices deep (the loads of
// slice i + 2 issued while slice i is computed and stored); a deeper one
// measured no faster.  Row pointers are uniform (scalar registers); a lane
// adds one offset.  Measured at C2 against the previous slice-by-slice
// epilogue (a|b of one slice in flight while it was staged): 266-279 ->
// 258-265 us, bit-identical.
__device__ __forceinline__ void down_bwd_full_epilogue(const GemmArgs& args, const f32x4 (&acc)[core::FM][core::FN],
                                                       uint8_t* ep, int el, int64_t grow0, int col0) {
  using namespace core;
  uint4 dhv[FM][4];
  {
    const int r = el & 15;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        // chunk c of row r at slot c ^ r (256-byte rows)
        const int col = j * 16 + (el >> 4) * 4;
        const uint32_t off = r * 256 + ((((col >> 3) ^ r)) << 4) + (col & 7) * 2;
        *reinterpret_cast<uint2*>(ep + off) =
            make_uint2(pack2(acc[i][j][0], acc[i][j][1]), pack2(acc[i][j][2], acc[i][j][3]));
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int rr = t * 4 + (el >> 4), c = el & 15;
        dhv[i][t] = *reinterpret_cast<const uint4*>(ep + rr * 256 + ((c ^ rr) << 4));
      }
    }
  }
  // lane: rows 4 t + el / 16 of each slice, columns col0 + 8 (el % 16) .. +7
  const uint8_t* abase = reinterpret_cast<const uint8_t*>(args.aux + grow0 * args.ldaux + col0);
  const uint32_t aoff = static_cast<uint32_t>((el >> 4) * static_cast<int>(args.ldaux) + (el & 15) * 8) * 2u;
  const int64_t astep = args.ldaux * 2 * 4;  // bytes per 4 rows
  uint8_t* cbase = reinterpret_cast<uint8_t*>(args.c0 + grow0 * args.ldc0 + col0);
  const uint32_t coff = static_cast<uint32_t>((el >> 4) * static_cast<int>(args.ldc0) + (el & 15) * 8) * 2u;
  const int64_t cstep = args.ldc0 * 2 * 4;
  const int64_t binter = args.inter * 2;  // bytes from a to b (and from da to db)
  constexpr int kDepth = 2;               // slices of a|b loads in flight
  uint4 pa[FM][4], pb[FM][4];
  auto load_slice = [&](int i) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint8_t* rp = abase + (i * 4 + t) * astep;
      pa[i][t] = load16(reinterpret_cast<const uint16_t*>(rp + aoff), true);
      pb[i][t] = load16(reinterpret_cast<const uint16_t*>(rp + binter + aoff), true);
    }
  };
  asm volatile("" ::: "memory");  // the loads are not hoisted into the staging above
#pragma unroll
  for (int i = 0; i < kDepth; ++i) load_slice(i);
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    if (i > 0 && i + kDepth - 1 < FM) load_slice(i + kDepth - 1);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      uint4 dav, dbv;
      swiglu_bwd8(dhv[i][t], pa[i][t], pb[i][t], dav, dbv);
      uint8_t* rp = cbase + (i * 4 + t) * cstep;
      store16(reinterpret_cast<uint16_t*>(rp + coff), dav, true);
      store16(reinterpret_cast<uint16_t*>(rp + binter + coff), dbv, true);
    }
  }
}

// GATHER (GATEUP_FWD only): args.gather is set; a separate instantiation, so
// that the plain kernel carries none of the gathered path's code.
template <int MODE, bool GATHER = false>
__global__ __launch_bounds__(core::NT, 1) void rows_gemm_kernel(const GemmArgs args,
                                                                 const int32_t* __restrict__ offsets) {
  using namespace core;
  constexpr bool GA = MODE == GATEUP_FWD && GATHER;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w / WN, wn = w % WN;
  const uint32_t sbase = lds_addr(smem);

  // GATEUP_FWD: a tile covers 128 h columns (128 rows of w1 and of w3).
  constexpr int TN_COLS = (MODE == GATEUP_FWD) ? BN / 2 : BN;
  // The backward dX products read the weights as they lie ([K, N]) with
  // transposing LDS reads.
  constexpr bool BTR = (MODE == DOWN_BWD || MODE == GATEUP_BWD);
  const int tiles_n = (args.N + TN_COLS - 1) / TN_COLS;
  const int total_tiles = count_tiles(args, offsets, tiles_n);
  const int NP = static_cast<int>(gridDim.x), b = xcd_slot(static_cast<int>(blockIdx.x), NP);
  const int nk = args.K / BK;
  const SplitPlan sp = split_plan<MODE>(args, total_tiles, NP, nk);
  {
    // descriptors of the split tiles for the split reduction (after the
    // partials): first row, valid rows, first output column, valid columns
    // (GATEUP_FWD: h columns, 128 per tile)
    if (args.split_ws != nullptr && threadIdx.x == 0) {
      int4* hdr = reinterpret_cast<int4*>(args.split_ws + static_cast<int64_t>(NP) * BM * BN);
      const int r = static_cast<int>(blockIdx.x);
      if (r == 0) hdr[0] = make_int4(sp.R, sp.S, 0, 0);
      if (r < sp.R) {
        int g, tm, tn, row_base, M;
        locate_tile(args, offsets, tiles_n, sp.full + r, g, tm, tn, row_base, M);
        hdr[1 + r] = make_int4(row_base + tm * BM, min(M - tm * BM, BM), tn * TN_COLS,
                               min(args.N - tn * TN_COLS, TN_COLS));
      }
    }
  }
  const int my_items = (sp.items() - b + NP - 1) / NP;  // items b, b + NP, ...
  if (my_items <= 0) return;
  int total = 0;  // K steps of 64 over all of this workgroup's items
  for (int i = 0; i < my_items; ++i) {
    int t_, k0_, kn_, s_;
    split_item(sp, nk, b + i * NP, t_, k0_, kn_, s_);
    total += kn_;
  }

  // ---- global -> LDS copy cursor
  // Copy instruction i of wave w writes LDS rows 64 i + 8 w .. +7 of an operand;
  // lane l fetches row 64 i + drow, global chunk dchunk (the swizzled slot l % 8).
  const int drow = w * 8 + (lane >> 3);
  const int dchunk = (lane & 7) ^ swzk(drow);  // swzk(64 i + drow) == swzk(drow)
  // B as it lies (BTR): k row 16 i + drow_b, chunk cb_t (wsw(16 i + drow_b) == wsw(drow_b))
  const int drow_b = 2 * w + (lane >> 5);
  const int cb_t = ((((lane & 31) >> 1) ^ wsw(drow_b)) << 1) | (lane & 1);
  const uint32_t lds_copy = sbase + w * 1024;
  int c_ti = 0, c_kt = 0, c_k0 = 0, c_kn = 0;  // item ordinal, step within it, its K range
  const uint16_t* c_a = nullptr;   // A rows of the tile being copied
  const uint16_t* c_b0 = nullptr;  // B operand base(s)
  const uint16_t* c_b1 = nullptr;
  int c_last_row = 0, c_n0 = 0;    // last valid A row of the tile, first B row
  // GA: this lane's byte offsets (from c_a) of its A rows of the tile, rows
  // 64 i + drow clamped to the last valid one; the routed rows are token rows
  // of x (row r: x row gather[r] / gather_k).  The lane's four indices of an
  // item are loaded when the item before it is set up (g_pf, vector loads
  // issued after that stage's copies, complete by the next stage's wait) and
  // consumed one item later.
  uint32_t a_off[LA];
  int32_t g_pf[LA] = {0, 0, 0, 0};
  bool g_pf_routed = false;  // the prefetched item is a routed tile (its rows are gathered)
  auto item_rows = [&](int ti, int& row0, int& last, bool& routed) {
    int tile, k0_, kn_, slot;
    split_item(sp, nk, b + ti * NP, tile, k0_, kn_, slot);
    int g, tm, tn, row_base, M;
    routed = locate_tile(args, offsets, tiles_n, tile, g, tm, tn, row_base, M) && g < args.E;
    row0 = row_base + tm * BM;
    last = min(M - tm * BM, BM) - 1;
  };
  auto prefetch_rows = [&](int ti) {
    // item ti's indices (no loads past the last item or for the shared group)
    g_pf_routed = false;
    if (ti >= my_items) return;
    int row0, last;
    item_rows(ti, row0, last, g_pf_routed);
    if (!g_pf_routed) return;
#pragma unroll
    for (int i = 0; i < LA; ++i) {
      const uint32_t off = static_cast<uint32_t>(row0 + min(64 * i + drow, last)) * 4u;
      asm volatile("global_load_dword %0, %1, %2" : "+v"(g_pf[i]) : "v"(off), "s"(args.gather) : "memory");
    }
  };
  auto copy_tile = [&](int ti) {
    int tile, slot;
    split_item(sp, nk, b + ti * NP, tile, c_k0, c_kn, slot);
    int g, tm, tn, row_base, M;
    locate_tile(args, offsets, tiles_n, tile, g, tm, tn, row_base, M);
    const bool gathered = GA && g < args.E;
    const uint16_t* A = gathered ? args.a_routed
                        : (g < args.E || args.a_shared == nullptr) ? args.a_routed + static_cast<int64_t>(row_base) * args.lda
                                                                   : args.a_shared;
    c_a = gathered ? A : A + static_cast<int64_t>(tm) * BM * args.lda;
    c_last_row = min(M - tm * BM, BM) - 1;
    c_b0 = args.b0[g];
    c_b1 = args.b1[g];
    c_n0 = tn * TN_COLS;
    if constexpr (GA) {
      if (gathered) {
        // g_pf holds this item's indices (loaded one item ahead, a stage wait
        // has normally passed since; the wait here covers every operation older
        // than this stage's LT copies and orders the use after it)
        asm volatile("s_waitcnt vmcnt(%4)"
                     : "+v"(g_pf[0]), "+v"(g_pf[1]), "+v"(g_pf[2]), "+v"(g_pf[3])
                     : "n"(LT)
                     : "memory");
#pragma unroll
        for (int i = 0; i < LA; ++i) {
          const uint32_t tok = slot_token(static_cast<uint32_t>(g_pf[i]), args.gather_magic);
          a_off[i] = (tok * static_cast<uint32_t>(args.lda) + static_cast<uint32_t>(dchunk * 8)) * 2u;
        }
      } else {
#pragma unroll
        for (int i = 0; i < LA; ++i)
          a_off[i] = static_cast<uint32_t>(min(64 * i + drow, c_last_row) * static_cast<int>(args.lda) + dchunk * 8) * 2u;
      }
      prefetch_rows(ti + 1);
    }
  };
  if constexpr (GA) {
    // the first item's indices, waited for at once
    prefetch_rows(0);
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(g_pf[0]), "+v"(g_pf[1]), "+v"(g_pf[2]), "+v"(g_pf[3])::"memory");
  }
  copy_tile(0);
  const int lda = static_cast<int>(args.lda), ldb = static_cast<int>(args.ldb);
  auto issue = [&](int it) {
    const uint32_t st = lds_copy + (it & 1) * STAGE;
    const int kofs = (c_k0 + c_kt) * BK;
    auto copy_a = [&]() {
#pragma unroll
      for (int i = 0; i < LA; ++i) {
        if constexpr (GA) {
          copy16(st + i * 8192, c_a + kofs, a_off[i]);
        } else {
          const int r = min(64 * i + drow, c_last_row);
          copy16(st + i * 8192, c_a + kofs, static_cast<uint32_t>(r * lda + dchunk * 8) * 2u);
        }
      }
    };
    auto copy_b = [&]() {
      if constexpr (BTR) {
        // 64 k rows of 512 bytes: instruction i of wave w writes k rows 16 i + 2 w, +1;
        // lane l: k row 16 i + drow_b, logical 16-byte chunk cb_t (32-byte windows
        // swizzled by wsw(k row)).  GATEUP_BWD: k < inter from w1, else from w3.
        const uint16_t* bb = (MODE == GATEUP_BWD && kofs >= args.inter)
                                 ? c_b1 + static_cast<int64_t>(kofs - args.inter) * args.ldb
                                 : c_b0 + static_cast<int64_t>(kofs) * args.ldb;
        const int col = min(c_n0 + 8 * cb_t, args.N - 8);
#pragma unroll
        for (int i = 0; i < LB; ++i)
          copy16(st + A_BYTES + i * 8192, bb, static_cast<uint32_t>((16 * i + drow_b) * ldb + col) * 2u);
      } else {
#pragma unroll
        for (int i = 0; i < LB; ++i) {
          // GATEUP_FWD bands: w1 rows (even i) and w3 rows (odd i), 64 h columns each
          const int n = min(c_n0 + ((MODE == GATEUP_FWD) ? (i >> 1) * 64 : 64 * i) + drow, args.N - 1);
          const uint16_t* b = (MODE == GATEUP_FWD && (i & 1)) ? c_b1 : c_b0;
          copy16(st + A_BYTES + i * 8192, b + kofs, static_cast<uint32_t>(n * ldb + dchunk * 8) * 2u);
        }
      }
    };
    // The dX products issue the weight rows first (512-byte rows of a matrix
    // that every CU streams) and the activation rows after them: gate/up dX
    // 289 -> 283 us at C2, the down backward within noise; in the forward
    // products the order made no difference (same instructions and waits).
    if constexpr (BTR) {
      copy_b();
      copy_a();
    } else {
      copy_a();
      copy_b();
    }
    if (++c_kt == c_kn) {
      c_kt = 0;
      if (++c_ti < my_items) copy_tile(c_ti);
    }
  };

  // ---- fragment address bases (A rows / B rows of this wave; BTR: trb_base)
  uint32_t xa = frag_base(wm * WTM, lane);
  uint32_t xb = BTR ? trb_base(wn, lane) : frag_base(wn * WTN, lane);

  issue(0);
  if (total > 1) {
    issue(1);
    wait_vm_barrier<LT>();
  } else {
    wait_vm_barrier<0>();
  }
  bf16x8 P[FN], Q[2][4];
#pragma unroll
  for (int p = 0; p < FN; ++p)
    P[p] = BTR ? trb_frag(sbase + (xb ^ (static_cast<uint32_t>(p) << 5)))
               : *reinterpret_cast<const bf16x8*>(smem + A_BYTES + (xb + 2048u * p));
#pragma unroll
  for (int q = 0; q < 4; ++q) Q[0][q] = *reinterpret_cast<const bf16x8*>(smem + (xa + 2048u * q));
  // Q[1] is a read-write operand of the first block8 statements (overwritten
  // there by their ds_reads): give it a defined value.
#pragma unroll
  for (int q = 0; q < 4; ++q) Q[1][q] = Q[0][q];

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  uint8_t* ep = smem + 2 * STAGE + w * EPI;  // this wave's epilogue staging (4 KB)
  int e_ti = 0, e_kt = 0, e_kn = c_kn, e_slot = -1, e_tile = 0;
  {
    int k0_;
    split_item(sp, nk, b, e_tile, k0_, e_kn, e_slot);
  }
  int last_epi = -4;        // iteration whose end wrote an epilogue
  bool last_full = false;   // that epilogue issued exactly epi_stores<MODE>() stores
  for (int it = 0; it < total; ++it) {
    // keep the per-step fragment addresses from being hoisted out of the loop
    asm volatile("" : "+v"(xa), "+v"(xb));
    const uint32_t cur = sbase + (it & 1) * STAGE;
    if constexpr (BTR)
      kstep_t<1>(acc, P, Q[0], Q[1], xa, xb, cur);
    else
      kstep<64>(acc, P, Q[0], Q[1], xa, xb, cur);  // reads the second K half of this stage
    uint32_t src = cur;                           // the last step re-reads (harmlessly) its own stage
    if (it + 1 < total) {
      // Stage (it+1) must have landed; stage it&1 is free once every wave is past
      // this point.  Stores of an epilogue written after copy it+1 was issued may
      // still be in flight (only when their number is exact).
      if (it - last_epi == 1 && last_full)
        wait_vm_barrier<epi_stores<MODE>()>();
      else
        wait_vm_barrier<0>();
      if (it + 2 < total) issue(it + 2);
      src = sbase + ((it + 1) & 1) * STAGE;
    }
    if constexpr (BTR)
      kstep_t<0>(acc, P, Q[1], Q[0], xa, xb, src);
    else
      kstep<0>(acc, P, Q[1], Q[0], xa, xb, src);

    if (++e_kt < e_kn) continue;
    // ---- tile epilogue: this wave's 64 x 128 block
    e_kt = 0;
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3\n" ::: "memory");  // MFMA results -> VALU reads
    // lane index as an opaque value: keeps the epilogue's address arithmetic
    // from being hoisted out of the main loop (where it would occupy registers)
    int el = lane;
    asm volatile("" : "+v"(el));
    if (e_slot >= 0) {
      // K-split range: fp32 partial of the 256 x 256 tile (local row-major)
      float* part = args.split_ws + static_cast<int64_t>(e_slot) * BM * BN;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          *reinterpret_cast<f32x4*>(part + (wm * WTM + i * 16 + (el & 15)) * BN + wn * WTN + j * 16 + (el >> 4) * 4) =
              acc[i][j];
    } else {
      int g, tm, tn, row_base, M;
      locate_tile(args, offsets, tiles_n, e_tile, g, tm, tn, row_base, M);
      const int rows_valid = min(M - tm * BM, BM);
      const int col0 = tn * TN_COLS + wn * (TN_COLS / WN);  // first output column of this wave
      const bool full = rows_valid == BM && (tn + 1) * TN_COLS <= args.N;
      const int64_t grow0 = static_cast<int64_t>(row_base) + tm * BM + wm * WTM;
      bool epi_done = false;
      if constexpr (MODE == DOWN_BWD) {
        if (full) {
          down_bwd_full_epilogue(args, acc, ep, el, grow0, col0);
          epi_done = true;
        }
      }
      if (!epi_done)
  #pragma unroll
      for (int i = 0; i < FM; ++i) {
        // DOWN_BWD (partial tiles; full ones took down_bwd_full_epilogue): a|b
        // of the 16 rows go in flight before the staging below, all 8 loads at
        // once (rows and columns clamped into the tile, so the addresses stay
        // valid for a partial tile; such values are not stored)
        uint4 pa[4], pb[4];
        if constexpr (MODE == DOWN_BWD) {
  #pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int r = t * 4 + (el >> 4), c = el & 15;
            const int64_t growc = grow0 - wm * WTM + min(wm * WTM + i * 16 + r, rows_valid - 1);
            const uint16_t* src = args.aux + growc * args.ldaux + min(col0 + c * 8, args.N - 8);
            pa[t] = load16(src, true);
            pb[t] = load16(src + args.inter, true);
          }
        }
        // stage rows 16 i .. 16 i + 15 of the wave block, 128 accumulator columns
        // (256 bytes per row; chunk c of row r at slot c ^ r); GATEUP_FWD keeps
        // the packed a | b values for h below
        uint2 pk[FN];
        {
          const int r = el & 15;
  #pragma unroll
          for (int j = 0; j < FN; ++j) {
            const int col = j * 16 + (el >> 4) * 4;
            const uint32_t off = r * 256 + ((((col >> 3) ^ r)) << 4) + (col & 7) * 2;
            pk[j].x = pack2(acc[i][j][0], acc[i][j][1]);
            pk[j].y = pack2(acc[i][j][2], acc[i][j][3]);
            *reinterpret_cast<uint2*>(ep + off) = pk[j];
          }
        }
  #pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int r = t * 4 + (el >> 4), c = el & 15;
          const uint4 v = *reinterpret_cast<const uint4*>(ep + r * 256 + ((c ^ r) << 4));
          const int lrow = wm * WTM + i * 16 + r;
          const int64_t grow = grow0 + i * 16 + r;
          if constexpr (MODE == GATEUP_FWD) {
            // columns 0..63: a, 64..127: b for h columns col0 .. col0 + 63
            const int hc = col0 + (c & 7) * 8;
            if (full || (lrow < rows_valid && hc < args.N)) {
              store16(args.c0 + grow * args.ldc0 + (c < 8 ? 0 : args.inter) + hc, v, true);
            }
          } else if constexpr (MODE == DOWN_BWD) {
            // h = s * b, s = bf16(silu(a)); dh arrives bf16-rounded:
            // da = bf16(bf16(dh * b) * silu'(a)), db = bf16(dh * s)
            const int hc = col0 + c * 8;
            if (full || (lrow < rows_valid && hc < args.N)) {
              uint4 dav, dbv;
              swiglu_bwd8(v, pa[t], pb[t], dav, dbv);
              store16(args.c0 + grow * args.ldc0 + hc, dav, true);
              store16(args.c0 + grow * args.ldc0 + args.inter + hc, dbv, true);
            }
          } else {
            const int oc = col0 + c * 8;
            if (full || (lrow < rows_valid && oc < args.N))
              *reinterpret_cast<uint4*>(args.c0 + grow * args.ldc0 + oc) = v;
          }
        }
        if constexpr (MODE == GATEUP_FWD) {
          // h = bf16(bf16(silu(a)) * b) for the 16 rows x 64 h columns, staged as
          // 128-byte rows (chunk c of row r at slot c ^ swz(r))
          const int r = el & 15;
  #pragma unroll
          for (int j = 0; j < 4; ++j) {
            // a = bf16(acc) and b likewise, as staged above
            const float a[4] = {__uint_as_float(pk[j].x << 16), __uint_as_float(pk[j].x & 0xffff0000u),
                                __uint_as_float(pk[j].y << 16), __uint_as_float(pk[j].y & 0xffff0000u)};
            const float b[4] = {__uint_as_float(pk[j + 4].x << 16), __uint_as_float(pk[j + 4].x & 0xffff0000u),
                                __uint_as_float(pk[j + 4].y << 16), __uint_as_float(pk[j + 4].y & 0xffff0000u)};
            float hv[4];
  #pragma unroll
            for (int e = 0; e < 4; ++e) hv[e] = a[e] * fast_sigmoid(a[e]);
            bf_round2(hv[0], hv[1]);
            bf_round2(hv[2], hv[3]);
  #pragma unroll
            for (int e = 0; e < 4; ++e) hv[e] = hv[e] * b[e];
            const int col = j * 16 + (el >> 4) * 4;
            const uint32_t off = r * 128 + ((((col >> 3) ^ swz(r))) << 4) + (col & 7) * 2;
            uint2 v;
            v.x = pack2(hv[0], hv[1]);
            v.y = pack2(hv[2], hv[3]);
            *reinterpret_cast<uint2*>(ep + off) = v;
          }
  #pragma unroll
          for (int t = 0; t < 2; ++t) {
            const int rr = t * 8 + (el >> 3), c = el & 7;
            const uint4 v = *reinterpret_cast<const uint4*>(ep + rr * 128 + ((c ^ swz(rr)) << 4));
            const int lrow = wm * WTM + i * 16 + rr;
            const int hc = col0 + c * 8;
            if (full || (lrow < rows_valid && hc < args.N))
              store16(args.c1 + (grow0 + i * 16 + rr) * args.ldc1 + hc, v, true);
          }
        }
      }
      last_full = full;
    }  // whole tile
    if (e_slot >= 0) last_full = false;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    asm volatile("s_nop 1" ::: "memory");  // VALU writes -> MFMA reads of the accumulators
    last_epi = it;
    if constexpr (MODE == DOWN_BWD) {
      // The fragments the last K step read for the next tile are read again
      // (its first stage has landed, waited for above; after the last tile
      // the reads harmlessly re-read a stage), so that their registers are
      // free during the epilogue, which needs them for the a|b loads (no
      // branch in the K loop: a K step that skipped the reads before an
      // epilogue kept both sets live and spilled).
      const uint32_t nst = sbase + ((it + 1) & 1) * STAGE;
      typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;
#pragma unroll
      for (int p = 0; p < FN; ++p) P[p] = trb_frag(nst + (xb ^ (static_cast<uint32_t>(p) << 5)));
#pragma unroll
      for (int q = 0; q < 4; ++q) Q[0][q] = *(const lds_bf16x8*)(uintptr_t)(nst + xa + 2048u * q);
    }
    if (++e_ti < my_items) {
      int k0_;
      split_item(sp, nk, b + e_ti * NP, e_tile, k0_, e_kn, e_slot);
    }
  }
}

// ---- split reductions
// The product wrote, after the P tiles of partials, a header {R, S} and one
// descriptor {first row, valid rows, first output column, valid output
// columns} per split tile.  A reduction sums a split tile's S partials in
// range order and writes the tile through the product's epilogue.  Block =
// (split tile r, sixteenth of its rows); a thread takes units of 8
// consecutive partial columns of one row.  Every partial slot is a whole
// BM x BN region, so the loads need no bounds; only valid rows and columns
// are stored.

struct SplitTile {
  bool active;
  int S;
  int4 d;
  const float* src0;  // the tile's first partial
};

__device__ __forceinline__ SplitTile split_tile(const float* ws, int P) {
  using namespace core;
  const int4* hdr = reinterpret_cast<const int4*>(ws + static_cast<int64_t>(P) * BM * BN);
  const int4 h0 = hdr[0];
  const int r = blockIdx.x / kReduceParts;
  SplitTile t;
  t.active = r < h0.x;
  t.S = h0.y;
  t.d = t.active ? hdr[1 + r] : make_int4(0, 0, 0, 0);
  t.src0 = ws + static_cast<int64_t>(r) * h0.y * BM * BN;
  return t;
}

// Partial values o .. o + 7 of the S ranges, summed in range order from 0
// (all kSplitMaxS loads issued first; ranges past S re-read range S - 1 and
// are not added).
__device__ __forceinline__ void sum_ranges8(const SplitTile& t, int o, float* acc) {
  using namespace core;
  float4 u[kSplitMaxS][2];
#pragma unroll
  for (int s = 0; s < kSplitMaxS; ++s) {
    const float* p = t.src0 + static_cast<int64_t>(min(s, t.S - 1)) * BM * BN + o;
    u[s][0] = *reinterpret_cast<const float4*>(p);
    u[s][1] = *reinterpret_cast<const float4*>(p + 4);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
#pragma unroll
  for (int s = 0; s < kSplitMaxS; ++s) {
    const float v[8] = {u[s][0].x, u[s][0].y, u[s][0].z, u[s][0].w, u[s][1].x, u[s][1].y, u[s][1].z, u[s][1].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = (s < t.S) ? acc[e] + v[e] : acc[e];
  }
}

// DOWN_FWD, GATEUP_BWD: the bf16 tile.  Two units per thread.
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* __restrict__ ws, int P,
                                                           uint16_t* __restrict__ out, int64_t ldo) {
  using namespace core;
  const SplitTile t = split_tile(ws, P);
  if (!t.active) return;
  const int row0 = (blockIdx.x % kReduceParts) * 16;
  float acc[2][8];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int u = threadIdx.x + q * 256;
    sum_ranges8(t, (row0 + u / 32) * BN + (u % 32) * 8, acc[q]);
  }
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int u = threadIdx.x + q * 256, row = row0 + u / 32, col = (u % 32) * 8;
    if (row < t.d.y && col < t.d.w)
      *reinterpret_cast<uint4*>(out + static_cast<int64_t>(t.d.x + row) * ldo + t.d.z + col) = pack8(acc[q]);
  }
}

// GATEUP_FWD: a|b = bf16(acc), h = bf16(bf16(silu(a)) * b), as the tile
// epilogue.  The partial columns of wave half w hold a for h columns
// 64 w .. 64 w + 63, then b for the same columns.  One unit per thread.
__global__ __launch_bounds__(256) void split_reduce_gateup_kernel(const GemmArgs args, int P) {
  using namespace core;
  const SplitTile t = split_tile(args.split_ws, P);
  if (!t.active) return;
  const int row = (blockIdx.x % kReduceParts) * 16 + threadIdx.x / 16, hc = (threadIdx.x % 16) * 8;
  const int pa = (hc / 64) * 128 + hc % 64;
  float a[8], b[8];
  sum_ranges8(t, row * BN + pa, a);
  sum_ranges8(t, row * BN + pa + 64, b);
  if (row >= t.d.y || hc >= t.d.w) return;
  const uint4 pka = pack8(a), pkb = pack8(b);
  const int64_t grow = static_cast<int64_t>(t.d.x) + row;
  const int col = t.d.z + hc;
  store16(args.c0 + grow * args.ldc0 + col, pka, true);
  store16(args.c0 + grow * args.ldc0 + args.inter + col, pkb, true);
  float ar[8], br[8], hv[8];
  unpack8(pka, ar);
  unpack8(pkb, br);
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    float h0v = ar[e] * fast_sigmoid(ar[e]), h1v = ar[e + 1] * fast_sigmoid(ar[e + 1]);
    bf_round2(h0v, h1v);
    hv[e] = h0v * br[e];
    hv[e + 1] = h1v * br[e + 1];
  }
  store16(args.c1 + grow * args.ldc1 + col, pack8(hv), true);
}

// DOWN_BWD: dh = bf16(acc), then the SwiGLU backward of the tile epilogue
// with a|b read from args.aux (rows and columns clamped into the tile for
// the loads).  Two units per thread.
__global__ __launch_bounds__(256) void split_reduce_down_bwd_kernel(const GemmArgs args, int P) {
  using namespace core;
  const SplitTile t = split_tile(args.split_ws, P);
  if (!t.active) return;
  const int row0 = (blockIdx.x % kReduceParts) * 16;
  float acc[2][8];
  uint4 la[2], lb[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int u = threadIdx.x + q * 256, row = row0 + u / 32, c = (u % 32) * 8;
    const int64_t lrow = static_cast<int64_t>(t.d.x) + min(row, t.d.y - 1);
    const uint16_t* src = args.aux + lrow * args.ldaux + t.d.z + min(c, t.d.w - 8);
    la[q] = load16(src, true);
    lb[q] = load16(src + args.inter, true);
    sum_ranges8(t, row * BN + c, acc[q]);
  }
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int u = threadIdx.x + q * 256, row = row0 + u / 32, c = (u % 32) * 8;
    if (row >= t.d.y || c >= t.d.w) continue;
    const int64_t grow = static_cast<int64_t>(t.d.x) + row;
    const int hc = t.d.z + c;
    uint4 dav, dbv;
    swiglu_bwd8(pack8(acc[q]), la[q], lb[q], dav, dbv);  // dh arrives bf16-rounded, as in the tile epilogue
    store16(args.c0 + grow * args.ldc0 + hc, dav, true);
    store16(args.c0 + grow * args.ldc0 + args.inter + hc, dbv, true);
  }
}

// ---- small groups (decode-sized batches) -------------------------------------
// A group of at most kSmallM rows would leave a 256 x 256 tile nearly empty
// and run its whole K loop in one workgroup; such a product is bound by
// streaming the weights, so the aim is to have all of them in flight at once.
// One workgroup owns 16 output columns of one group (GATEUP_FWD: 16 h
// columns, i.e. the same 16 rows of w1 and of w3, two accumulators); its
// waves (4 for the gate/up product, 8 for the down product, whose K is the
// longer one in the reference's shapes: the faster counts measured) split
// the K steps of 32 evenly, and each wave issues the loads of up to CH steps
// before their MFMAs (v_mfma_f32_16x16x32_bf16, operands read straight from
// memory: the weights once, the few activation rows from L2).  The partial
// tiles are added in wave order through LDS.  MB = 16-row blocks the kernel is built for (the
// host picks it from a bound on the group sizes; with MB > 2 fewer K steps
// are in flight, the activation fragments take the registers; a group of
// more than 16 MB rows runs as slabs of 16 MB rows); a slab that needs fewer
// blocks runs the 2- or 4-block variant, with more K steps in flight.  Rows past a group's end repeat its last row and are not stored.
constexpr int kSmallM = 128;
// The host knows the shared expert's row count, so the small kernel takes the
// shared group as slabs of kSharedSlab rows in workgroups of their own (more
// workgroups, each with more K steps of loads in flight).
constexpr int kSharedSlab = 64;

template <int MODE>
constexpr int small_waves() { return MODE == GATEUP_FWD ? 4 : 8; }

template <int MODE>
constexpr int small_nb() { return MODE == GATEUP_FWD ? 2 : 1; }  // weight matrices
constexpr int kSmallPass = 2;  // m blocks reduced per LDS pass

// One slab of at most 16 MB rows of one group: the K loop with CH steps of
// loads in flight, then the wave-order reduction through LDS and the stores.
// The MFMA chain of every accumulator runs over the wave's K steps in order,
// whatever MB and CH are, so the result does not depend on them.
template <int MODE, int MB>
__device__ __forceinline__ void small_slab(const GemmArgs& args,
                                           float (*red)[kSmallPass][small_nb<MODE>()][4][64], int wave,
                                           int lane, int cb, const uint16_t* A, int M, int row_base,
                                           const uint16_t* w0, const uint16_t* w1, int s_begin, int s_end) {
  constexpr int kSmallWaves = small_waves<MODE>();
  constexpr int NB = small_nb<MODE>();
  constexpr int CH = MB <= 2 ? 8 : (MB == 4 ? 4 : 2);
  constexpr int PASS = kSmallPass;
  const int r16 = lane & 15, kq = (lane >> 4) * 8;
  const int mb_n = (M + 15) / 16;  // 1 .. MB
  const uint16_t* ap[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
    ap[mb] = A + static_cast<int64_t>(min(16 * mb + r16, M - 1)) * args.lda + kq;

  f32x4 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[mb][b] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
  for (int s0 = s_begin; s0 < s_end; s0 += CH) {
    bf16x8 bw[CH][NB], af[CH][MB];
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      if (s0 + u < s_end) {
        const int k = 32 * (s0 + u);
        bw[u][0] = *reinterpret_cast<const bf16x8*>(w0 + k);
        if constexpr (NB == 2) bw[u][1] = *reinterpret_cast<const bf16x8*>(w1 + k);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          if (mb < mb_n) af[u][mb] = *reinterpret_cast<const bf16x8*>(ap[mb] + k);
      }
    }
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      if (s0 + u < s_end) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          if (mb < mb_n)
#pragma unroll
            for (int b = 0; b < NB; ++b)
              acc[mb][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bw[u][b], af[u][mb], acc[mb][b], 0, 0, 0);
      }
    }
  }
  // Passes of PASS m blocks: every wave parks its partials, wave p of the pass
  // adds the eight partials of m block (pass base + p) in wave order and stores.
  const int m = lane & 15, n0 = cb * 16 + (lane >> 4) * 4;
  for (int base = 0; base < mb_n; base += PASS) {
#pragma unroll
    for (int p = 0; p < PASS; ++p) {
      const int mb = base + p;
#pragma unroll
      for (int q = 0; q < MB; ++q)  // static register index
        if (q == mb)
#pragma unroll
          for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wave][p][b][r][lane] = acc[q][b][r];
    }
    __syncthreads();
    const int mb = base + wave;
    if (wave < PASS && mb < mb_n && 16 * mb + m < M) {
      float v[NB][4];
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float t = red[0][wave][b][r][lane];
#pragma unroll
          for (int w = 1; w < kSmallWaves; ++w) t = t + red[w][wave][b][r][lane];
          v[b][r] = t;
        }
      const int64_t row = row_base + 16 * mb + m;
      if constexpr (MODE == GATEUP_FWD) {
        float hv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          v[0][r] = bf_round(v[0][r]);
          v[1][r] = bf_round(v[1][r]);
          hv[r] = bf_round(v[0][r] * fast_sigmoid(v[0][r])) * v[1][r];
        }
        uint16_t* ab = args.c0 + row * args.ldc0;
        *reinterpret_cast<uint2*>(ab + n0) = make_uint2(pack2(v[0][0], v[0][1]), pack2(v[0][2], v[0][3]));
        *reinterpret_cast<uint2*>(ab + args.inter + n0) =
            make_uint2(pack2(v[1][0], v[1][1]), pack2(v[1][2], v[1][3]));
        *reinterpret_cast<uint2*>(args.c1 + row * args.ldc1 + n0) =
            make_uint2(pack2(hv[0], hv[1]), pack2(hv[2], hv[3]));
      } else {
        *reinterpret_cast<uint2*>(args.c0 + row * args.ldc0 + n0) =
            make_uint2(pack2(v[0][0], v[0][1]), pack2(v[0][2], v[0][3]));
      }
    }
    __syncthreads();
  }
}

// The 2- and 4-block variants are held to 3 (gate/up) or 4 (down) waves per
// SIMD, one more than the compiler picks by itself, without spills: a
// decode launch of a few thousand waves then needs fewer rounds (C3 M = 32:
// gate/up 15.8 -> 14.1 us, down 13.0 -> 11.6 us).  The 1-block variant is
// faster without the bound, the 8-block gate/up variant would spill.
template <int MODE, int MB>
__global__ __launch_bounds__(small_waves<MODE>() * 64)
__attribute__((amdgpu_waves_per_eu((MB == 2 || MB == 4) ? (MODE == GATEUP_FWD ? 3 : 4) : 1))) void small_gemm_kernel(
    const GemmArgs args) {
  static_assert(MODE == GATEUP_FWD || MODE == DOWN_FWD, "forward products only");
  constexpr int kSmallWaves = small_waves<MODE>();
  __shared__ float red[kSmallWaves][kSmallPass][small_nb<MODE>()][4][64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ncb = args.N / 16;
  const int cb = blockIdx.x % ncb;
  int g, row_base, M, shared_off = 0;
  if (MODE == DOWN_FWD && args.small_compact) {
    // Fewer routed rows than experts: workgroup -> (group, column block) over
    // the groups this kernel takes (1 .. small_max rows: routed experts in
    // order, then the shared expert), so that the grid holds no workgroups
    // of empty experts (empty 8-wave workgroups ahead of the busy ones cost
    // up to 2 us at M = 1).  Lane e < E reads expert e's rows, the wave ranks
    // the qualifying experts with a ballot and takes the rank-th.
    const int rank = blockIdx.x / ncb, lane_e = threadIdx.x & 63;
    int lo = 0, m_e = 0;
    if (lane_e < args.E) {
      lo = args.offsets[lane_e];
      m_e = args.offsets[lane_e + 1] - lo;
    }
    const bool qual = m_e > 0 && m_e <= args.small_max;
    const uint64_t qmask = __ballot(qual);
    const int nq = __popcll(qmask);
    if (rank < nq) {
      const uint64_t below = lane_e == 0 ? 0ull : (qmask & (~0ull >> (64 - lane_e)));
      g = __ffsll(static_cast<unsigned long long>(__ballot(qual && __popcll(below) == rank))) - 1;
      row_base = __shfl(lo, g, 64);
      M = __shfl(m_e, g, 64);
    } else {
      // the shared expert, slab rank - nq
      shared_off = (rank - nq) * kSharedSlab;
      if (args.rows_shared > args.small_max || shared_off >= args.rows_shared) return;
      g = args.E;
      row_base = args.rows_routed + shared_off;
      M = min(kSharedSlab, args.rows_shared - shared_off);
    }
  } else {
    // one workgroup per (routed group or shared slab, column block); empty
    // groups return at once
    g = blockIdx.x / ncb;
    if (g < args.E) {
      row_base = args.offsets[g];
      M = args.offsets[g + 1] - row_base;
      if (M == 0 || M > args.small_max) return;
    } else {
      shared_off = (g - args.E) * kSharedSlab;
      if (args.rows_shared > args.small_max || shared_off >= args.rows_shared) return;
      g = args.E;
      row_base = args.rows_routed + shared_off;
      M = min(kSharedSlab, args.rows_shared - shared_off);
    }
  }
  const uint16_t* A_group = (g < args.E || args.a_shared == nullptr)
                                ? args.a_routed + static_cast<int64_t>(row_base) * args.lda
                                : args.a_shared + static_cast<int64_t>(shared_off) * args.lda;
  // Fragments (operands swapped: srcA = weight rows, srcB = activation rows):
  // lane l supplies row l % 16 of each, K elements 8 (l / 16) .. +7 of a step,
  // and gets C[m = l % 16][n = 4 (l / 16) + 0..3].
  const int r16 = lane & 15, kq = (lane >> 4) * 8;
  const uint16_t* w0 = args.b0[g] + static_cast<int64_t>(cb * 16 + r16) * args.ldb + kq;
  const uint16_t* w1 = (MODE == GATEUP_FWD) ? args.b1[g] + static_cast<int64_t>(cb * 16 + r16) * args.ldb + kq
                                            : nullptr;
  const int nsteps = args.K / 32;
  const int s_begin = wave * nsteps / kSmallWaves, s_end = (wave + 1) * nsteps / kSmallWaves;
  // A group of more than 16 MB rows (at most small_max = 2 kSmallM) runs as
  // slabs of 16 MB rows, each streaming the weights again.
  const int M_group = M, row_base_group = row_base;
  for (int slab = 0; slab < M_group; slab += 16 * MB) {
    const int M = min(16 * MB, M_group - slab), row_base = row_base_group + slab;
    const uint16_t* A = A_group + static_cast<int64_t>(slab) * args.lda;
    const int mb_n = (M + 15) / 16;  // 1 .. MB
    // A launch built for MB blocks runs a smaller slab with fewer blocks and
    // more K steps in flight.
    if constexpr (MB >= 4) {
      if (mb_n <= 2) {
        small_slab<MODE, 2>(args, red, wave, lane, cb, A, M, row_base, w0, w1, s_begin, s_end);
        continue;
      }
    }
    if constexpr (MB >= 8) {
      if (mb_n <= 4) {
        small_slab<MODE, 4>(args, red, wave, lane, cb, A, M, row_base, w0, w1, s_begin, s_end);
        continue;
      }
    }
    small_slab<MODE, MB>(args, red, wave, lane, cb, A, M, row_base, w0, w1, s_begin, s_end);
  }
}

// ---- weight gradients (K-grouped) -------------------------------------------
// G_e = A_e^T B_e with A_e [M_e, m_out], B_e [M_e, n_out] (both MN-contiguous).
// Work unit = (group, K chunk of kc rows, output tile).  A group whose rows fit
// in one chunk writes its tile directly; otherwise every chunk writes an fp32
// partial and wgrad_reduce_kernel adds the chunks of a group in chunk order.
struct WgradArgs {
  const uint16_t* a_routed;
  const uint16_t* a_shared;
  int64_t lda;
  const uint16_t* b_routed;  // [rows_routed, n_out], or with b_gather: x [T, n_out]
  const uint16_t* b_shared;
  int64_t ldb;
  const int32_t* b_gather;   // routed row r of B is b_routed row b_gather[r] / gather_k (nullptr: row r)
  int gather_k;
  uint64_t gather_magic;     // slot_div_magic(gather_k)
  const int32_t* offsets;
  int E;
  int rows_routed;
  int rows_shared;
  int m_out, n_out, m_split;
  int kc;
  int out_dtype;
  float* partial;
  void* out_lo[FMOE_MAX_EXPERTS + 1];
  void* out_hi[FMOE_MAX_EXPERTS + 1];
};

__device__ __forceinline__ void group_rows(const WgradArgs& a, int g, int& row_base, int& M) {
  if (g < a.E) {
    row_base = a.offsets[g];
    M = a.offsets[g + 1] - row_base;
  } else {
    row_base = a.rows_routed;
    M = a.rows_shared;
  }
}

// ---- weight gradients on the shared core ------------------------------------
// Both operands are MN-contiguous ([rows, m_out] and [rows, n_out]), so their
// 64 x 256 stage tiles are copied as they lie in memory (K-major: 64 k rows of
// 512 bytes) with the same global -> LDS copies as the row products, and the
// MFMA fragments are read with ds_read_b64_tr_b16, which returns to lane
// (h = l / 16, i = l % 16) of each 16-lane group the i-th column of the 4 x 4
// block of 16-bit values that source lanes 4 j + q address (row j, 4 values at
// column 4 q): two such reads give a lane 8 consecutive k of one output row.
// The 32-byte windows of a k row are XOR-swizzled by wsw(row) so that the 16
// rows x 32 bytes a read instruction touches fall on distinct banks.
using core::wsw;

typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ bf16x8 tr_frag(uint32_t addr) {
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uintptr_t)addr);
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uintptr_t)(addr + 2048u));
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// GATHER: args.b_gather is set (a separate instantiation, so that the plain
// kernel carries none of the gathered path's code).
template <bool GATHER>
__global__ __launch_bounds__(core::NT, 1) void wgrad_tr_kernel(const WgradArgs args,
                                                               const int32_t* __restrict__ offsets) {
  using namespace core;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * STAGE];
  // Gathered B rows: the slot indices of each stage's 64 k rows (ring of eight
  // stages, filled by global -> LDS copies three stages ahead and read one
  // stage ahead, after the stage waits that cover them; a slot is refilled
  // four stages after its last read, with stage barriers in between).
  __shared__ int32_t idx_ring[8][BK];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w / WN, wn = w % WN;  // wave block: 64 m x 128 n
  const uint32_t sbase = lds_addr(smem);
  const int tiles_m = (args.m_out + BM - 1) / BM, tiles_n = (args.n_out + BN - 1) / BN;
  const int tiles = tiles_m * tiles_n;
  const int G = args.E + (args.rows_shared > 0 ? 1 : 0);

  // ---- work unit -> (group, K chunk, output tile).  Units are dispatched in
  // order (largest groups' chunks first when they come first); the hardware
  // hands the next unit to the next free CU, which balances the uneven units.
  int unit = blockIdx.x;
  int g = 0, row_base = 0, M = 0, chunks = 0, pbase = 0;
  for (; g < G; ++g) {
    if (g < args.E) {
      const int2 o = core::sload2(offsets + g);
      row_base = o.x;
      M = o.y - o.x;
    } else {
      row_base = args.rows_routed;
      M = args.rows_shared;
    }
    chunks = (M + args.kc - 1) / args.kc;
    const int nu = chunks * tiles;
    if (unit < nu) break;
    unit -= nu;
    if (chunks > 1) pbase += chunks;
  }
  if (g >= G) return;
  const int chunk = unit / tiles, tile = unit - chunk * tiles;
  int tm = tile / tiles_n, tn = tile - tm * tiles_n;
  if (tiles % 8 == 0) {
    // A chunk's units start at a multiple of 8, so workgroup b runs on XCD
    // tile % 8 (workgroups go to the 8 XCDs round-robin).  Each XCD takes whole
    // column blocks of one operand (its L2 then serves them to all of that
    // XCD's tiles of the chunk) and the same share of every chunk.
    const int xcd = tile & 7, j = tile >> 3;
    if (tiles_m % 8 == 0) {
      tm = xcd + 8 * (j / tiles_n);
      tn = j % tiles_n;
    } else if (tiles_n % 8 == 0) {
      tn = xcd + 8 * (j / tiles_m);
      tm = j % tiles_m;
    }
  }
  const int m0 = tm * BM, n0 = tn * BN;
  const int k_begin = chunk * args.kc;
  const int k_end = min(M, k_begin + args.kc);
  const int nk = (k_end - k_begin + BK - 1) / BK;
  const bool shared_sep = (g >= args.E);
  const uint16_t* A = (shared_sep && args.a_shared) ? args.a_shared : args.a_routed + static_cast<int64_t>(row_base) * args.lda;
  const bool gathered = GATHER && !shared_sep;
  const uint16_t* B = (shared_sep && args.b_shared) ? args.b_shared
                      : gathered ? args.b_routed
                                 : args.b_routed + static_cast<int64_t>(row_base) * args.ldb;
  const int lda = static_cast<int>(args.lda), ldb = static_cast<int>(args.ldb);
  const uint32_t ring = lds_addr(&idx_ring[0][0]);
  // stage kt's slot indices into ring slot kt % 8 (wave 0; rows past k_end
  // repeat the last valid one)
  auto fetch_idx = [&](int kt) {
    if (w == 0) {
      const int r = min(k_begin + kt * BK + lane, k_end - 1);
      copy4(ring + (kt & 7) * (BK * 4), args.b_gather + row_base, static_cast<uint32_t>(r) * 4u);
    }
  };
  // ---- copies: instruction i of wave w writes k rows 16 i + drow (1 KB = 2 rows of 512 B);
  // lane chunk p = l % 32 holds logical chunk c of the row
  const int drow = 2 * w + (lane >> 5);
  const int p = lane & 31;
  const int c = (((p >> 1) ^ wsw(drow)) << 1) | (p & 1);  // wsw(16 i + drow) == wsw(drow)
  const int colA = min(m0 + 8 * c, args.m_out - 8), colB = min(n0 + 8 * c, args.n_out - 8);
  const uint32_t lds_copy = sbase + w * 1024;
  uint32_t b_off[4];  // gathered B: this lane's byte offsets (from B) of its 4 k rows of a coming stage
  auto form_offsets = [&](int kt) {
    const int last = k_end - 1 - (k_begin + kt * BK);  // >= 0 for kt < nk
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = min(16 * i + drow, last);
      const uint32_t tok = slot_token(static_cast<uint32_t>(idx_ring[kt & 7][r]), args.gather_magic);
      b_off[i] = (tok * static_cast<uint32_t>(ldb) + static_cast<uint32_t>(colB)) * 2u;
    }
  };
  if (gathered) {
    // stages 0..2 before the first copies (issue(kt) fetches stage kt + 3)
    for (int q = 0; q < 3 && q < nk; ++q) fetch_idx(q);
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  }

  auto issue = [&](int kt) {
    const int k0 = k_begin + kt * BK;
    const int last = k_end - 1 - k0;  // last valid k row of this stage
    const uint32_t st = lds_copy + (kt & 1) * STAGE;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = min(16 * i + drow, last);
      copy16(st + i * 8192, A + static_cast<int64_t>(k0) * lda, static_cast<uint32_t>(r * lda + colA) * 2u);
    }
    if (gathered) {
      // k row r of the stage is x row (slot of group row k0 + r) / k, at the
      // offsets b_off formed from the stage's ring slot (at the end of the K
      // step before, or before the first copies)
#pragma unroll
      for (int i = 0; i < 4; ++i) copy16(st + A_BYTES + i * 8192, B, b_off[i]);
      if (kt + 3 < nk) fetch_idx(kt + 3);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = min(16 * i + drow, last);
        copy16(st + A_BYTES + i * 8192, B + static_cast<int64_t>(k0) * ldb,
               static_cast<uint32_t>(r * ldb + colB) * 2u);
      }
    }
  };
  // Rows past k_end in a stage hold copies of the last valid row: zero their A
  // side (after this wave's copies have landed) so that they add nothing.
  auto zero_tail = [&](int kt) {
    const int k0 = k_begin + kt * BK;
    if (k_end - k0 >= BK) return;
    uint8_t* st = smem + (kt & 1) * STAGE + w * 1024 + lane * 16;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (k0 + 16 * i + drow >= k_end) *reinterpret_cast<uint4*>(st + i * 8192) = make_uint4(0, 0, 0, 0);
  };
  auto sync_stage = [&](int kt, bool more_in_flight) {
    if (more_in_flight) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    zero_tail(kt);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };

  // ---- fragment addresses: lane (h, s = 4 jq + q); window swizzle fr = wsw(8 h + jq)
  const int h = lane >> 4, jq = (lane >> 2) & 3, q = lane & 3;
  const int fr = jq | ((h & 1) << 2);
  const uint32_t xa = static_cast<uint32_t>((8 * h + jq) * 512 + (((4 * wm) ^ fr) << 5) + 8 * q);
  const uint32_t xb = static_cast<uint32_t>(A_BYTES + (8 * h + jq) * 512 + ((8 * wn + fr) << 5) + 8 * q);

  if (gathered) form_offsets(0);
  issue(0);
  if (nk > 1) {
    if (gathered) form_offsets(1);
    issue(1);
  }
  if (gathered) form_offsets(min(2, nk - 1));
  sync_stage(0, nk > 1);

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  bf16x8 fa[FM], fb[FN];
#pragma unroll
  for (int f = 0; f < FM; ++f) fa[f] = tr_frag(sbase + (xa ^ (f << 5)));
#pragma unroll
  for (int f = 0; f < FN; ++f) fb[f] = tr_frag(sbase + (xb ^ (f << 5)));

  for (int kt = 0; kt < nk; ++kt) {
    const uint32_t cur = sbase + (kt & 1) * STAGE;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      uint32_t src = cur + 16384u;  // second K half of this stage
      if (ks == 1) {
        src = cur;  // the last step re-reads (harmlessly) its own stage
        if (kt + 1 < nk) {
          sync_stage(kt + 1, false);
          if (kt + 2 < nk) issue(kt + 2);
          src = sbase + ((kt + 1) & 1) * STAGE;
        }
      }
      bf16x8 na[FM], nb[FN];
#pragma unroll
      for (int f = 0; f < FM; ++f) na[f] = tr_frag(src + (xa ^ (f << 5)));
#pragma unroll
      for (int f = 0; f < FN; ++f) nb[f] = tr_frag(src + (xb ^ (f << 5)));
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[j], fa[i], acc[i][j], 0, 0, 0);
      // interleave: per 8 MFMAs, 6 fragment reads (24 reads, 32 MFMAs per step)
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
#pragma unroll
      for (int f = 0; f < FM; ++f) fa[f] = na[f];
#pragma unroll
      for (int f = 0; f < FN; ++f) fb[f] = nb[f];
    }
    // gathered B: the offsets of stage kt + 3 (issued in the next K step),
    // formed after this step's MFMAs rather than right after a barrier,
    // where every wave would wait for its ring reads at once.  The ring slot
    // landed before this step's second wait; past the last stage the last
    // one is formed again (unused).
    if (gathered) form_offsets(min(kt + 3, nk - 1));
  }

  // ---- epilogue: lane holds C[m0 + 64 wm + 16 i + l % 16][n0 + 128 wn + 16 j + 4 (l / 16) + 0..3]
  const int64_t mn = static_cast<int64_t>(args.m_out) * args.n_out;
  float* part = (chunks > 1) ? args.partial + static_cast<int64_t>(pbase + chunk) * mn : nullptr;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int m = m0 + wm * WTM + i * 16 + (lane & 15);
    if (m >= args.m_out) continue;
    const bool lo = m < args.m_split;
    void* base = lo ? args.out_lo[g] : args.out_hi[g];
    const int64_t orow = static_cast<int64_t>(lo ? m : m - args.m_split) * args.n_out;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = n0 + wn * WTN + j * 16 + (lane >> 4) * 4;
      if (n >= args.n_out) continue;
      const f32x4 v = acc[i][j];
      if (part) {
        *reinterpret_cast<f32x4*>(part + static_cast<int64_t>(m) * args.n_out + n) = v;
      } else if (args.out_dtype == FMOE_BF16) {
        uint2 u;
        u.x = pack2(v[0], v[1]);
        u.y = pack2(v[2], v[3]);
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(base) + orow + n) = u;
      } else {
        *reinterpret_cast<f32x4*>(static_cast<float*>(base) + orow + n) = v;
      }
    }
  }
}

// Adds the chunk partials of each multi-chunk group in chunk order; 8
// consecutive outputs of one row per thread (m_out and n_out are multiples of
// 64), written with 16-byte stores.  The loads of kWgradReduceBatch chunks are
// issued together (a loop that waited for each chunk's loads before the next
// paid one memory latency per chunk); the sums still run in chunk order,
// from 0.  A group without rows gets a zero gradient (no work unit of the
// product kernel writes it).
constexpr int kWgradReduceBatch = 8;

__device__ __forceinline__ void store_grad8(const WgradArgs& a, int g, int64_t i0, const float (&v)[8]) {
  const int m = static_cast<int>(i0 / a.n_out), n = static_cast<int>(i0 - static_cast<int64_t>(m) * a.n_out);
  const bool lo = m < a.m_split;
  const int64_t o = static_cast<int64_t>(lo ? m : m - a.m_split) * a.n_out + n;
  void* base = lo ? a.out_lo[g] : a.out_hi[g];
  if (a.out_dtype == FMOE_BF16) {
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(base) + o) = pack8(v);
  } else {
    float4* dst = reinterpret_cast<float4*>(static_cast<float*>(base) + o);
    dst[0] = make_float4(v[0], v[1], v[2], v[3]);
    dst[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
}

__global__ __launch_bounds__(256) void wgrad_reduce_kernel(const WgradArgs args) {
  const int g = blockIdx.y;
  int row_base, M;
  group_rows(args, g, row_base, M);
  const int chunks = (M + args.kc - 1) / args.kc;
  const int64_t mn = static_cast<int64_t>(args.m_out) * args.n_out;
  const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 8;
  if (i0 >= mn || chunks == 1) return;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (chunks > 1) {
    int pbase = 0;
    for (int q = 0; q < g; ++q) {
      int rb, Mq;
      group_rows(args, q, rb, Mq);
      const int cq = (Mq + args.kc - 1) / args.kc;
      if (cq > 1) pbase += cq;
    }
    const float* src0 = args.partial + static_cast<int64_t>(pbase) * mn + i0;
    for (int c0 = 0; c0 < chunks; c0 += kWgradReduceBatch) {
      float4 u[kWgradReduceBatch][2];
#pragma unroll
      for (int b = 0; b < kWgradReduceBatch; ++b) {
        // chunks past the last re-read the last one and are not added
        const float4* src = reinterpret_cast<const float4*>(src0 + min(c0 + b, chunks - 1) * mn);
        u[b][0] = src[0];
        u[b][1] = src[1];
      }
#pragma unroll
      for (int b = 0; b < kWgradReduceBatch; ++b) {
        if (c0 + b < chunks) {
          acc[0] = acc[0] + u[b][0].x; acc[1] = acc[1] + u[b][0].y;
          acc[2] = acc[2] + u[b][0].z; acc[3] = acc[3] + u[b][0].w;
          acc[4] = acc[4] + u[b][1].x; acc[5] = acc[5] + u[b][1].y;
          acc[6] = acc[6] + u[b][1].z; acc[7] = acc[7] + u[b][1].w;
        }
      }
    }
  }
  store_grad8(args, g, i0, acc);
}

// ---- host side --------------------------------------------------------------
int check_common(int n_experts, int64_t rows_routed, int64_t rows_shared, int64_t dim, int64_t inter) {
  if (n_experts <= 0 || n_experts > FMOE_MAX_EXPERTS) return FMOE_ERR_TOO_MANY_EXPERTS;
  if (rows_routed < 0 || rows_shared < 0 || dim <= 0 || inter <= 0) return FMOE_ERR_INVALID_ARG;
  if (dim % 64 != 0 || inter % 64 != 0) return FMOE_ERR_SHAPE;
  if (rows_routed + rows_shared > INT32_MAX / 2) return FMOE_ERR_SHAPE;
  return FMOE_OK;
}

// The four row products.  Their tile copies address a lane's operand row
// with a 32-bit byte offset from the tile's base: up to 255 rows of at most
// 2 * inter (or dim) elements for the activations, any row of the weight for
// the forward products (n * K + 56 < dim * inter elements).  So a row holds
// fewer than 2^22 elements and a weight matrix fewer than 2^31.
int check_row_product(int n_experts, int64_t rows_routed, int64_t rows_shared, int64_t dim, int64_t inter) {
  const int st = check_common(n_experts, rows_routed, rows_shared, dim, inter);
  if (st) return st;
  constexpr int64_t kMaxRow = int64_t(1) << 22;
  if (dim >= kMaxRow || inter >= kMaxRow || dim * inter >= (int64_t(1) << 31)) return FMOE_ERR_SHAPE;
  return FMOE_OK;
}

// Row counts up to which a launch sends groups of <= kSmallM rows to the
// small-group kernel (decode-sized batches); larger launches use the tiled
// kernel for every group.
constexpr int64_t kSmallLaunchRows = 4096;

// Compute units of the current device (the persistent grid size), cached per
// device ordinal.
int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
  cache[dev].store(v, std::memory_order_relaxed);
  return v;
}

// 16-row blocks of the small-group kernel for a launch whose groups have at
// most max_rows rows (1, 2, 4 or 8; the down product stops at 4, so that
// its larger groups run as 64-row slabs: measured faster, as its 8-block
// variant holds fewer waves per SIMD).
template <int MODE>
inline int small_blocks(int64_t max_rows) {
  const int64_t mb = ceil_div(max_rows < kSmallM ? max_rows : kSmallM, 16);
  return mb <= 1 ? 1 : mb <= 2 ? 2 : (mb <= 4 || MODE == DOWN_FWD) ? 4 : 8;
}

template <int MODE>
int launch_rows(GemmArgs& a, int64_t rows_routed, int64_t rows_shared, int E, void* stream) {
  constexpr int TN_COLS = (MODE == GATEUP_FWD) ? core::BN / 2 : core::BN;
  const int64_t tiles_n = ceil_div(a.N, TN_COLS);
  constexpr bool kHasSmall = (MODE == GATEUP_FWD || MODE == DOWN_FWD);
  a.small_max = (kHasSmall && rows_routed + rows_shared <= kSmallLaunchRows) ? kSmallM : 0;
  // A routed group has at most rows_routed rows: when no group can exceed
  // 2 kSmallM rows (the small kernel takes a larger group as two slabs), the
  // tiled kernel (and its split reduction) would have nothing to do.  This
  // is the case for a decode step of up to 128 tokens at top-2, whose groups
  // the host cannot bound more tightly.
  const bool all_small = a.small_max > 0 && rows_routed <= 2 * kSmallM && rows_shared <= kSmallM;
  if (all_small) a.small_max = 2 * kSmallM;
  // Upper bound of sum over groups of ceil(M_g / BM): floor(rows/BM) + groups.
  const int64_t tiles = (rows_routed / core::BM + E + ceil_div(rows_shared, core::BM)) * tiles_n;
  if (tiles <= 0) return FMOE_OK;
  if (!all_small) {
    const int64_t grid = tiles < device_cus() ? tiles : device_cus();
    // A run of kSplitMaxRounds full rounds or more never splits (split_plan);
    // sum over groups of ceil(M_g / BM) >= ceil(rows / BM) bounds the tile
    // count from below, so such a run skips the header and the reduction.
    const int64_t tiles_lo = (ceil_div(rows_routed, core::BM) + ceil_div(rows_shared, core::BM)) * tiles_n;
    if (a.small_max == 0 && tiles_lo / grid >= kSplitMaxRounds) a.split_ws = nullptr;
    bool gathered = false;
    if constexpr (MODE == GATEUP_FWD) {
      gathered = a.gather != nullptr;
      if (gathered) rows_gemm_kernel<MODE, true><<<dim3(grid), dim3(core::NT), 0, as_stream(stream)>>>(a, a.offsets);
    }
    if (!gathered) rows_gemm_kernel<MODE, false><<<dim3(grid), dim3(core::NT), 0, as_stream(stream)>>>(a, a.offsets);
    if (a.split_ws != nullptr) {
      if constexpr (MODE == DOWN_FWD || MODE == GATEUP_BWD)
        split_reduce_kernel<<<dim3(grid * kReduceParts), dim3(256), 0, as_stream(stream)>>>(
            a.split_ws, static_cast<int>(grid), a.c0, a.ldc0);
      else if constexpr (MODE == GATEUP_FWD)
        split_reduce_gateup_kernel<<<dim3(grid * kReduceParts), dim3(256), 0, as_stream(stream)>>>(
            a, static_cast<int>(grid));
      else
        split_reduce_down_bwd_kernel<<<dim3(grid * kReduceParts), dim3(256), 0, as_stream(stream)>>>(
            a, static_cast<int>(grid));
    }
  }
  if constexpr (kHasSmall) {
    if (a.small_max > 0) {
      // DOWN_FWD with fewer routed rows than experts: the grid covers the
      // at most rows_routed routed groups that have rows
      a.small_compact = (MODE == DOWN_FWD && rows_routed < E) ? 1 : 0;
      const int64_t Gr = a.small_compact ? rows_routed : E;
      const int64_t shared_slabs =
          (rows_shared > 0 && rows_shared <= a.small_max) ? ceil_div(rows_shared, kSharedSlab) : 0;
      const int64_t G = Gr + shared_slabs;
      if (G == 0) return launch_status();
      const dim3 grid(G * (a.N / 16)), block(small_waves<MODE>() * 64);
      hipStream_t s = as_stream(stream);
      const int64_t shared_bound = rows_shared < kSharedSlab ? rows_shared : kSharedSlab;
      switch (small_blocks<MODE>(rows_routed > shared_bound ? rows_routed : shared_bound)) {
        case 1: small_gemm_kernel<MODE, 1><<<grid, block, 0, s>>>(a); break;
        case 2: small_gemm_kernel<MODE, 2><<<grid, block, 0, s>>>(a); break;
        case 4: small_gemm_kernel<MODE, 4><<<grid, block, 0, s>>>(a); break;
        default:
          if constexpr (MODE != DOWN_FWD) small_gemm_kernel<MODE, 8><<<grid, block, 0, s>>>(a);
          break;
      }
    }
  }
  return launch_status();
}

void fill_groups(GemmArgs& a, const int32_t* offsets, int E, int64_t rows_routed, int64_t rows_shared) {
  a.offsets = offsets;
  a.E = E;
  a.rows_routed = static_cast<int>(rows_routed);
  a.rows_shared = static_cast<int>(rows_shared);
}

}  // namespace fmoe

using namespace fmoe;

extern "C" size_t fmoe_split_workspace_bytes(void) {
  const size_t P = static_cast<size_t>(device_cus());
  return P * core::BM * core::BN * sizeof(float) + (P + 1) * 16;  // partials + descriptors
}

extern "C" int fmoe_gateup_fwd(const void* x_routed, const int32_t* gather, int gather_k, int64_t gather_tokens,
                               const void* x_shared, const int32_t* offsets,
                               int n_experts, int64_t rows_routed, int64_t rows_shared, int64_t dim,
                               int64_t inter, const void* const* w1, const void* const* w3,
                               void* ab, void* h, void* workspace, size_t workspace_bytes, void* stream) {
  int st = check_row_product(n_experts, rows_routed, rows_shared, dim, inter);
  if (st) return st;
  if (rows_routed + rows_shared == 0) return FMOE_OK;
  if (!offsets || !w1 || !w3 || !ab || !h || (rows_routed && !x_routed) ||
      (rows_shared && !x_shared))
    return FMOE_ERR_INVALID_ARG;
  if (!aligned16(ab) || !aligned16(h)) return FMOE_ERR_ALIGN;
  if (gather) {
    // routed row r reads x_routed ([gather_tokens, dim]) row gather[r] / gather_k;
    // the tiled kernel reads the indices in windows of 8 and forms 32-bit offsets
    if (gather_k <= 0 || gather_k > FMOE_MAX_TOPK || gather_tokens <= 0 || rows_routed < 8 ||
        rows_routed + rows_shared <= kSmallLaunchRows || gather_tokens * dim * 2 >= (int64_t(1) << 31) ||
        rows_routed >= (int64_t(1) << 29))
      return FMOE_ERR_SHAPE;
  }
  GemmArgs a = {};
  a.a_routed = static_cast<const uint16_t*>(x_routed);
  a.gather = gather;
  a.gather_k = gather ? gather_k : 1;
  a.gather_magic = slot_div_magic(a.gather_k);
  a.a_shared = static_cast<const uint16_t*>(x_shared);
  a.lda = dim;
  fill_groups(a, offsets, n_experts, rows_routed, rows_shared);
  a.K = static_cast<int>(dim);
  a.N = static_cast<int>(inter);
  a.inter = static_cast<int>(inter);
  a.ldb = dim;
  a.c0 = static_cast<uint16_t*>(ab);
  a.c1 = static_cast<uint16_t*>(h);
  a.ldc0 = 2 * inter;
  a.ldc1 = inter;
  a.split_ws = (workspace && workspace_bytes >= fmoe_split_workspace_bytes()) ? static_cast<float*>(workspace) : nullptr;
  const int G = n_experts + (rows_shared > 0 ? 1 : 0);
  for (int g = 0; g < G; ++g) {
    if (!w1[g] || !w3[g]) return FMOE_ERR_INVALID_ARG;
    a.b0[g] = static_cast<const uint16_t*>(w1[g]);
    a.b1[g] = static_cast<const uint16_t*>(w3[g]);
  }
  return launch_rows<GATEUP_FWD>(a, rows_routed, rows_shared, n_experts, stream);
}

extern "C" int fmoe_down_fwd(const void* h, const int32_t* offsets, int n_experts,
                             int64_t rows_routed, int64_t rows_shared, int64_t dim, int64_t inter,
                             const void* const* w2, void* out, void* workspace, size_t workspace_bytes,
                             void* stream) {
  int st = check_row_product(n_experts, rows_routed, rows_shared, dim, inter);
  if (st) return st;
  if (rows_routed + rows_shared == 0) return FMOE_OK;
  if (!h || !offsets || !w2 || !out) return FMOE_ERR_INVALID_ARG;
  if (!aligned16(out)) return FMOE_ERR_ALIGN;
  GemmArgs a = {};
  a.a_routed = static_cast<const uint16_t*>(h);
  a.a_shared = nullptr;
  a.lda = inter;
  fill_groups(a, offsets, n_experts, rows_routed, rows_shared);
  a.K = static_cast<int>(inter);
  a.N = static_cast<int>(dim);
  a.inter = static_cast<int>(inter);
  a.ldb = inter;
  a.c0 = static_cast<uint16_t*>(out);
  a.ldc0 = dim;
  a.split_ws = (workspace && workspace_bytes >= fmoe_split_workspace_bytes()) ? static_cast<float*>(workspace) : nullptr;
  const int G = n_experts + (rows_shared > 0 ? 1 : 0);
  for (int g = 0; g < G; ++g) {
    if (!w2[g]) return FMOE_ERR_INVALID_ARG;
    a.b0[g] = static_cast<const uint16_t*>(w2[g]);
  }
  return launch_rows<DOWN_FWD>(a, rows_routed, rows_shared, n_experts, stream);
}

extern "C" int fmoe_down_bwd_dx(const void* d_out_routed, const void* d_out_shared,
                                const int32_t* offsets, int n_experts, int64_t rows_routed,
                                int64_t rows_shared, int64_t dim, int64_t inter, const void* const* w2,
                                const void* ab, void* d_ab, void* workspace, size_t workspace_bytes,
                                void* stream) {
  int st = check_row_product(n_experts, rows_routed, rows_shared, dim, inter);
  if (st) return st;
  if (rows_routed + rows_shared == 0) return FMOE_OK;
  if (!offsets || !w2 || !ab || !d_ab || (rows_routed && !d_out_routed) ||
      (rows_shared && !d_out_shared))
    return FMOE_ERR_INVALID_ARG;
  if (!aligned16(ab) || !aligned16(d_ab)) return FMOE_ERR_ALIGN;
  GemmArgs a = {};
  a.a_routed = static_cast<const uint16_t*>(d_out_routed);
  a.a_shared = static_cast<const uint16_t*>(d_out_shared);
  a.lda = dim;
  fill_groups(a, offsets, n_experts, rows_routed, rows_shared);
  a.K = static_cast<int>(dim);
  a.N = static_cast<int>(inter);
  a.inter = static_cast<int>(inter);
  a.ldb = inter;  // w2[g] is [dim, inter] as nn.Linear keeps it: k row = dim index, inter contiguous
  a.c0 = static_cast<uint16_t*>(d_ab);
  a.ldc0 = 2 * inter;
  a.aux = static_cast<const uint16_t*>(ab);
  a.ldaux = 2 * inter;
  a.split_ws = (workspace && workspace_bytes >= fmoe_split_workspace_bytes()) ? static_cast<float*>(workspace) : nullptr;
  const int G = n_experts + (rows_shared > 0 ? 1 : 0);
  for (int g = 0; g < G; ++g) {
    if (!w2[g]) return FMOE_ERR_INVALID_ARG;
    if (!aligned16(w2[g])) return FMOE_ERR_ALIGN;
    a.b0[g] = static_cast<const uint16_t*>(w2[g]);
  }
  return launch_rows<DOWN_BWD>(a, rows_routed, rows_shared, n_experts, stream);
}

extern "C" int fmoe_gateup_bwd_dx(const void* d_ab, const int32_t* offsets, int n_experts,
                                  int64_t rows_routed, int64_t rows_shared, int64_t dim,
                                  int64_t inter, const void* const* w1, const void* const* w3, void* dx_rows,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  int st = check_row_product(n_experts, rows_routed, rows_shared, dim, inter);
  if (st) return st;
  if (rows_routed + rows_shared == 0) return FMOE_OK;
  if (!d_ab || !offsets || !w1 || !w3 || !dx_rows) return FMOE_ERR_INVALID_ARG;
  if (!aligned16(d_ab) || !aligned16(dx_rows)) return FMOE_ERR_ALIGN;
  GemmArgs a = {};
  a.a_routed = static_cast<const uint16_t*>(d_ab);
  a.a_shared = nullptr;
  a.lda = 2 * inter;
  fill_groups(a, offsets, n_experts, rows_routed, rows_shared);
  a.K = static_cast<int>(2 * inter);
  a.N = static_cast<int>(dim);
  a.inter = static_cast<int>(inter);
  a.ldb = dim;  // w1[g], w3[g] are [inter, dim]: k rows 0..inter-1 from w1, inter.. from w3
  a.c0 = static_cast<uint16_t*>(dx_rows);
  a.ldc0 = dim;
  a.split_ws = (workspace && workspace_bytes >= fmoe_split_workspace_bytes()) ? static_cast<float*>(workspace) : nullptr;
  const int G = n_experts + (rows_shared > 0 ? 1 : 0);
  for (int g = 0; g < G; ++g) {
    if (!w1[g] || !w3[g]) return FMOE_ERR_INVALID_ARG;
    if (!aligned16(w1[g]) || !aligned16(w3[g])) return FMOE_ERR_ALIGN;
    a.b0[g] = static_cast<const uint16_t*>(w1[g]);
    a.b1[g] = static_cast<const uint16_t*>(w3[g]);
  }
  return launch_rows<GATEUP_BWD>(a, rows_routed, rows_shared, n_experts, stream);
}

namespace fmoe {
// Rows per K chunk of the weight gradient.  A work unit is (group, chunk,
// output tile); the chunk is sized so that the largest unit is about half of
// one CU's average share (tiles * rows / 64 K-steps over 256 CUs), which keeps
// the skewed groups (one or two experts holding most rows) from leaving a long
// tail.  A multiple of 64, at least 256 rows.
int64_t wgrad_kc(int64_t rows_routed, int64_t rows_shared, int64_t m_out, int64_t n_out) {
  const int64_t rows = rows_routed + rows_shared;
  const int64_t tiles = ceil_div(m_out, 256) * ceil_div(n_out, 256);
  int64_t kc = (tiles * rows / 512) / 64 * 64;
  return kc < 256 ? 256 : kc;
}
}  // namespace fmoe

extern "C" size_t fmoe_weight_grad_workspace_bytes(int64_t rows_routed, int64_t rows_shared,
                                                   int n_experts, int64_t m_out, int64_t n_out) {
  if (rows_routed < 0 || rows_shared < 0 || n_experts <= 0 || m_out <= 0 || n_out <= 0) return 0;
  const int64_t kc = wgrad_kc(rows_routed, rows_shared, m_out, n_out);
  // sum over groups of ceil(M_g / kc) <= floor(rows / kc) + groups
  const int64_t chunks = (rows_routed + rows_shared) / kc + n_experts + 1;
  return static_cast<size_t>(chunks * m_out * n_out) * sizeof(float);
}

extern "C" int fmoe_weight_grad(const void* a_routed, const void* a_shared, int64_t lda,
                                const void* b_routed, const void* b_shared, int64_t ldb,
                                const int32_t* b_gather, int gather_k, int64_t gather_tokens,
                                const int32_t* offsets, int n_experts, int64_t rows_routed,
                                int64_t rows_shared, int64_t m_out, int64_t n_out, int64_t m_split,
                                void* const* out_lo, void* const* out_hi, int out_dtype,
                                void* workspace, size_t workspace_bytes, void* stream) {
  int st = check_common(n_experts, rows_routed, rows_shared, m_out, n_out);
  if (st) return st;
  if (out_dtype != FMOE_BF16 && out_dtype != FMOE_F32) return FMOE_ERR_DTYPE;
  if (m_split <= 0 || m_split > m_out) return FMOE_ERR_SHAPE;
  if (rows_routed + rows_shared == 0) return FMOE_OK;
  if (!offsets || !out_lo || (m_split < m_out && !out_hi) || (rows_routed && (!a_routed || !b_routed)))
    return FMOE_ERR_INVALID_ARG;
  if (lda % 8 != 0 || ldb % 8 != 0) return FMOE_ERR_ALIGN;
  // rows of at least m_out (n_out) elements; the stage copies address up to
  // 63 rows past a stage's first with a 32-bit byte offset
  if (lda < m_out || ldb < n_out || lda >= (int64_t(1) << 24) || ldb >= (int64_t(1) << 24))
    return FMOE_ERR_SHAPE;
  if (workspace_bytes < fmoe_weight_grad_workspace_bytes(rows_routed, rows_shared, n_experts, m_out, n_out))
    return FMOE_ERR_WORKSPACE;
  if (!workspace) return FMOE_ERR_INVALID_ARG;
  WgradArgs a = {};
  a.a_routed = static_cast<const uint16_t*>(a_routed);
  a.a_shared = static_cast<const uint16_t*>(a_shared);
  a.lda = lda;
  a.b_routed = static_cast<const uint16_t*>(b_routed);
  a.b_shared = static_cast<const uint16_t*>(b_shared);
  a.ldb = ldb;
  if (b_gather) {
    // routed row r of B is b_routed ([gather_tokens, n_out]) row b_gather[r] / gather_k
    if (gather_k <= 0 || gather_k > FMOE_MAX_TOPK || gather_tokens <= 0 ||
        gather_tokens * ldb * 2 >= (int64_t(1) << 31) || rows_routed >= (int64_t(1) << 29))
      return FMOE_ERR_SHAPE;
  }
  a.b_gather = b_gather;
  a.gather_k = b_gather ? gather_k : 1;
  a.gather_magic = slot_div_magic(a.gather_k);
  a.offsets = offsets;
  a.E = n_experts;
  a.rows_routed = static_cast<int>(rows_routed);
  a.rows_shared = static_cast<int>(rows_shared);
  a.m_out = static_cast<int>(m_out);
  a.n_out = static_cast<int>(n_out);
  a.m_split = static_cast<int>(m_split);
  a.kc = static_cast<int>(wgrad_kc(rows_routed, rows_shared, m_out, n_out));
  a.out_dtype = out_dtype;
  a.partial = static_cast<float*>(workspace);
  const int G = n_experts + (rows_shared > 0 ? 1 : 0);
  for (int g = 0; g < G; ++g) {
    if (!out_lo[g] || (m_split < m_out && !out_hi[g])) return FMOE_ERR_INVALID_ARG;
    if (!aligned16(out_lo[g]) || (m_split < m_out && !aligned16(out_hi[g]))) return FMOE_ERR_ALIGN;
    a.out_lo[g] = out_lo[g];
    a.out_hi[g] = (m_split < m_out) ? out_hi[g] : nullptr;
  }
  const int64_t tiles = ceil_div(m_out, core::BM) * ceil_div(n_out, core::BN);
  const int64_t max_chunks = (rows_routed + rows_shared) / a.kc + G;
  hipStream_t s = as_stream(stream);
  if (b_gather)
    wgrad_tr_kernel<true><<<dim3(max_chunks * tiles), dim3(core::NT), 0, s>>>(a, offsets);
  else
    wgrad_tr_kernel<false><<<dim3(max_chunks * tiles), dim3(core::NT), 0, s>>>(a, offsets);
  const int64_t mn = m_out * n_out;
  wgrad_reduce_kernel<<<dim3(ceil_div(mn, 256 * 8), G), dim3(256), 0, s>>>(a);
  return launch_status();
}
