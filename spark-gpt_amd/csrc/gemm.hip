// FP8 / bf16 MFMA GEMMs of the FP8 MLP block (gfx950, CDNA4).
//
// Every GEMM here is C[m, n] = sum_k A[m, k] * B[n, k]: both operands are
// K-contiguous rows in HBM, except that a weight gradient (K = tokens) may
// read either operand as the token-major activation its producer wrote,
// through transposing LDS reads (MainLoop TR_A / TR_B).  One work-group (256 threads = 4 waves, one wave
// per SIMD) computes a 256 x 256 output tile with the pipelined main loop of
// mainloop.h; each wave owns 128 x 128 as 4 x 4 blocks of 32 x 32 MFMA
// accumulators.
//
// MFMA: v_mfma_f32_32x32x64_f8f6f4 (e4m3/e5m2 chosen per operand) or
// v_mfma_f32_32x32x16_bf16.  The B fragment is passed as the instruction's
// first operand and the A fragment as its second, so each lane holds ONE A
// row (lane % 32) and, in a 32x32 block, 16 accumulators for B-tile rows
// 8*(v/4) + 4*(lane/32) + v%4, v = 0..15.  Within one instruction both
// operands use the same (lane-half, byte) -> k assignment, so any consistent
// placement of K inside a fragment gives the same dot product.
//
// Output-column permutation: the B tile is filled with its rows permuted
// (plain_col / paired_col below), so that accumulator v of block nb of the
// lane in half g is output column  base + 16*nb + v  -- 16 (and across blocks
// 64 or 32) consecutive columns per lane.  Every epilogue access is then a
// 16-byte vector; LDS staging remains only for the transposed copies.
#include "common.h"
#include "mainloop.h"
#include "scale.h"

namespace sfp8 {

// Logical tile lid -> (tm, tn): tile rows in groups of 8, walking the tile
// columns of a group before the next group, so a column of B tiles is reused
// from L2 across the group's A tiles.
SFP8_DEV void raster(int lid, int tiles_m, int tiles_n, int& tm, int& tn) {
  constexpr int G = 8;
  const int group = G * tiles_n;
  const int first_m = (lid / group) * G;
  const int gsz = (tiles_m - first_m) < G ? (tiles_m - first_m) : G;
  tm = first_m + (lid % group) % gsz;
  tn = (lid % group) / gsz;
}

// Work-groups are dispatched round-robin over the 8 XCDs (pid % 8): the
// logical index of work-group pid of nwg when each XCD (with its own L2)
// takes a contiguous run of logical indices (walked from its end with rev).
// A bijection of [0, nwg).
SFP8_DEV int xcd_run(int pid, int nwg, bool rev = false) {
  const int per = nwg >> 3, rem = nwg & 7;
  const int xcd = pid & 7;
  const int len = xcd < rem ? per + 1 : per;
  const int local = rev ? len - 1 - (pid >> 3) : (pid >> 3);
  return (xcd < rem) ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
}

// Work-group -> tile mapping: XCD-contiguous runs of logical tiles, rastered
// as above.  rev: each XCD walks its run backwards, so that a consumer of the
// previous kernel's output (run in the same order, forwards) reads the most
// recently written row blocks first, while they may still be in the memory-
// side cache.
SFP8_DEV void tile_coords(int pid, int nwg, int tiles_m, int tiles_n, int& tm, int& tn, bool rev = false) {
  raster(xcd_run(pid, nwg, rev), tiles_m, tiles_n, tm, tn);
}

// Split-K mapping of a 1-D grid of tiles * splits work-groups.  Work-groups
// are dispatched round-robin over the 8 XCDs (pid % 8); each XCD takes a
// contiguous run of the split-major order (split, tile), so the work-groups
// resident on one XCD read the same K range of A and B (one split, or two
// where a run crosses a split boundary) and share it in that XCD's L2.  With
// splits a multiple of 8 each XCD runs whole splits over every tile; with 2
// or 4 each split takes 8 / splits XCDs (1.5-2 % faster than split-major
// order over all XCDs at 4 and 2 splits).  Tiles of a split are rastered as
// in tile_coords.
// The grid may be padded past tiles * splits (wgrad_grid); padding work-groups
// get split = splits and do nothing.
SFP8_DEV void split_tile_coords(int pid, int nwg, int tiles_m, int tiles_n, int splits, int& tm, int& tn,
                                int& split) {
  const int tiles = tiles_m * tiles_n;
  const int lid = xcd_run(pid, nwg);
  split = lid / tiles;
  raster(lid % tiles, tiles_m, tiles_n, tm, tn);
}

// Output column (within the 256-column tile) held in B-tile row r, plain
// layout: wave column wn owns rows 128*wn.., lane half g of block nb element
// v (row 32*nb + 8*(v/4) + 4*g + v%4) gets column 128*wn + 64*g + 16*nb + v.
SFP8_DEV int plain_col(int r) {
  const int rl = r & 127;
  return (r & 128) + 64 * ((rl >> 2) & 1) + 16 * (rl >> 5) + 4 * ((rl >> 3) & 3) + (rl & 3);
}

// The same for a 64*NB-row B tile (NB blocks of 32 per wave): B row r holds
// column 32*NB*wn + 16*NB*g + 16*nb + v, so a lane's NB blocks cover 16*NB
// consecutive columns.  plain_col_nb<4> == plain_col.
template <int NB>
SFP8_DEV int plain_col_nb(int r) {
  const int wn = r / (32 * NB), rl = r % (32 * NB);
  return 32 * NB * wn + 16 * NB * ((rl >> 2) & 1) + 16 * (rl >> 5) + 4 * ((rl >> 3) & 3) + (rl & 3);
}

// Paired (gate/up) layout, 8 waves: rows 0..127 are gate, 128..255 up; wave
// column wn (0..3) owns rows 32*wn.. of each half (one block); column (within
// the 128-column half) 32*wn + 16*g + v.
SFP8_DEV int paired_col8(int r) {
  const int rl = r & 127;
  return 32 * (rl >> 5) + 16 * ((rl >> 2) & 1) + 4 * ((rl >> 3) & 3) + (rl & 3);
}

// Paired (gate/up) layout: rows 0..127 are gate, 128..255 up; wave column wn
// owns rows 64*wn.. of each half; column (within the 128-column half)
// 64*wn + 32*g + 16*nb + v.
SFP8_DEV int paired_col(int r) {
  const int rl = r & 63;
  return (r & 64) + 32 * ((rl >> 2) & 1) + 16 * (rl >> 5) + 4 * ((rl >> 3) & 3) + (rl & 3);
}

// Copy of an LDS tile (nrows rows of 64 * NP bytes, LDS row stride `stride`)
// into a K-slab matrix: 64-byte column block p of tile row r goes to
// dst + (c0 / 64 + p) * ldrows * 64 + (r0 + r) * 64.  Sixteen consecutive
// threads read one contiguous LDS row (no bank conflicts for NP = 4); the
// global writes are 256-byte runs of 4 rows per block.
template <int NP, int NT = 256>
SFP8_DEV void lds_rows_to_kslab(const uint8_t* lds, int nrows, int stride, uint8_t* dst, int64_t ldrows, int64_t r0,
                                int64_t c0) {
  const int total = nrows * NP * 4;
  for (int idx = threadIdx.x; idx < total; idx += NT) {
    const int ch = idx & 3, pb = (idx >> 2) % NP, r = idx / (4 * NP);
    *reinterpret_cast<intx4*>(dst + (c0 / 64 + pb) * ldrows * 64 + (r0 + r) * 64 + ch * 16) =
        *reinterpret_cast<const intx4*>(lds + r * stride + pb * 64 + ch * 16);
  }
}

SFP8_DEV void store16(void* p, const uint32_t (&w)[4]) {
  *reinterpret_cast<intx4*>(p) = intx4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
}

// Round 16 accumulators to bf16 (as fp32 values), after scaling by s.
SFP8_DEV void round16_bf16(const floatx16& a, float s, float (&o)[16]) {
#pragma unroll
  for (int v = 0; v < 16; v += 2) {
    const uint32_t p = pack2_bf16(a[v] * s, a[v + 1] * s);
    o[v] = __uint_as_float(p << 16);
    o[v + 1] = __uint_as_float(p & 0xffff0000u);
  }
}

// ---------------------------------------------------------------------------
// (a6) gate/up forward + SwiGLU epilogue (spark-gpt train.py:975-1016).
// Tile: 256 tokens x 128 intermediate columns; the B tile holds gate rows
// n0..n0+127 then up rows I+n0..I+n0+127 (paired layout), so a lane holds g and
// u of the same 32 consecutive columns.
constexpr int kEpiStride = 144;

// With a MoE plan (grouped experts): tile row tm of padded expert order,
// its expert's W8 at w8 + e * w_estride and weight scale wscale[e]; tile
// rows past the plan's count exit.
// 8 waves (two per SIMD): wave (wm, wn) owns tile rows 128*wm.. and the gate
// and up columns 32*wn.. (one 32-column block of each), so the serial
// epilogue of one wave overlaps the other's on the same SIMD.
__global__ __launch_bounds__(512, 1) void swiglu_fwd_kernel(
    const uint8_t* __restrict__ x8, const uint8_t* __restrict__ w8, int64_t T, int64_t D, int64_t I,
    const float* __restrict__ scale, const float* __restrict__ wscale, float* __restrict__ amax,
    uint8_t* __restrict__ gu8, uint8_t* __restrict__ h8, uint8_t* __restrict__ h8t, int64_t ldt,
    int tiles_m, int tiles_n, const int* __restrict__ plan, int64_t w_estride) {
  extern __shared__ __align__(16) uint8_t lds[];
  int tm, tn;
  tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
  if (plan) {
    const MoePlan P{plan};
    if (tm >= P.ntiles()) return;  // work-group uniform
    const int e = P.expert(tm);
    w8 += e * w_estride;
    wscale += e;
  }
  const int64_t m0 = (int64_t)tm * kTile, n0 = (int64_t)tn * 128;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  floatx16 acc[4][2];  // [tb][0] gate, [tb][1] up
  // K-slab operands: x8 [D/64][ldt][64], w8 [D/64][2I][64]; one K stage of
  // the tile is 256 contiguous rows of A and two runs of 128 rows of B
  MainLoop<false, kFmtE4M3, kFmtE4M3, true, 2, kStages, 0, false, false, 4>::run(
      lds, x8 + m0 * kStage, D * ldt - m0 * kStage, [=](int r) { return r * kStage; }, (int)(ldt * kStage), w8,
      D * 2 * I, [=](int r) { return ((r >> 7) * (int)I + (int)n0 + paired_col8(r)) * kStage; },
      (int)(2 * I * kStage), (int)(D / kStage), acc);
  // All scales are powers of two, so the dequantization factor commutes with
  // every rounding step: with gb, ub = bf16(acc) (unscaled),
  //   g = gb*deq, u = ub*deq, h = (g*sig(g))*u = hb*deq^2, hb = (gb*sig)*ub,
  //   gu8 = e4m3(g*q1) = e4m3(gb*(deq*q1)),  h8 = e4m3(hb*(deq^2*q2)),
  //   amax1 = deq*max(|gb|,|ub|),  amax2 = deq^2*max|hb|.
  // Rows past T are zero in x8 (K-slab padding): they add 0 to the amax and
  // 0 bytes to the padding of h8 and h8t.
  const float deq = 1.0f / (scale[0] * wscale[0]);
  const float c_exp = deq * -1.4426950408889634f;
  const float m1 = deq * scale[1], m2 = deq * deq * scale[2];
  const float inv1 = 1.0f / m1, inv2 = 1.0f / m2;
  const float bnd1 = kE4M3Max * inv1, bnd2 = kE4M3Max * inv2;
  // epilogue LDS: the tile's g8, u8 and h8 bytes (256 x 128 each), then the amax slots
  uint8_t* Gt = lds;
  uint8_t* Ut = lds + kTile * kEpiStride;
  uint8_t* Ht = lds + 2 * kTile * kEpiStride;
  float* red = reinterpret_cast<float*>(lds + 3 * kTile * kEpiStride);
  float m_gu = 0.f, m_h = 0.f;
  const int fr = lane & 31, g = lane >> 5;
  const int cb = 32 * wn + 16 * g;  // first of this lane's 16 columns
  // g, u (bf16-rounded, unscaled) and h of unit (tb, q): 4 columns
  auto unit = [&](int tb, int q, float (&gb)[4], float (&ub)[4], float (&hb)[4]) {
    // g, u rounded to bf16 as in the bf16 path (train.py:1006-1007)
#pragma unroll
    for (int e = 0; e < 4; e += 2) {
      const uint32_t pg = pack2_bf16(acc[tb][0][4 * q + e], acc[tb][0][4 * q + e + 1]);
      const uint32_t pu = pack2_bf16(acc[tb][1][4 * q + e], acc[tb][1][4 * q + e + 1]);
      gb[e] = __uint_as_float(pg << 16);
      gb[e + 1] = __uint_as_float(pg & 0xffff0000u);
      ub[e] = __uint_as_float(pu << 16);
      ub[e + 1] = __uint_as_float(pu & 0xffff0000u);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(gb[e] * c_exp));
      hb[e] = gb[e] * sg * ub[e];
    }
  };
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    const int row = 128 * wm + 32 * tb + fr;  // token within the tile
    uint32_t gw[4], uw[4], hw[4];
    bool bad = false;
    {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float gb[4], ub[4], hb[4];
        unit(tb, q, gb, ub, hb);
        // NaN-propagating maxima: inside the e4m3 range (after scaling) the
        // unclamped conversions are exact; otherwise the row block is redone
        float a = max3_nan(fabsf(gb[0]), fabsf(ub[0]), fabsf(gb[1]));
        a = max3_nan(a, fabsf(ub[1]), fabsf(gb[2]));
        a = max3_nan(a, fabsf(ub[2]), fabsf(gb[3]));
        a = __builtin_elementwise_maximum(a, fabsf(ub[3]));
        float b = max3_nan(fabsf(hb[0]), fabsf(hb[1]), fabsf(hb[2]));
        b = __builtin_elementwise_maximum(b, fabsf(hb[3]));
        bad |= !(a <= bnd1) | !(b <= bnd2);
        m_gu = fmaxf(m_gu, a);  // a NaN here is redone by the exact path
        m_h = fmaxf(m_h, b);
        const int k = q;
        gw[k] = pack4_e4m3_scaled_noclamp(gb[0], gb[1], gb[2], gb[3], inv1, 0u);
        uw[k] = pack4_e4m3_scaled_noclamp(ub[0], ub[1], ub[2], ub[3], inv1, 0u);
        hw[k] = pack4_e4m3_scaled_noclamp(hb[0], hb[1], hb[2], hb[3], inv2, 0u);
      }
    }
    if (__builtin_amdgcn_ballot_w64(bad)) {  // wave-uniform; NaN or out-of-range data only
      asm volatile("" ::: "memory");
      {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float gb[4], ub[4], hb[4];
          unit(tb, q, gb, ub, hb);
#pragma unroll
          for (int e = 0; e < 4; ++e) {  // amax over the non-NaN values
            m_gu = fmaxf(m_gu, fmaxf(fabsf(gb[e]), fabsf(ub[e])));
            m_h = fmaxf(m_h, fabsf(hb[e]));
          }
          const int k = q;
          gw[k] = fix_nan4(pack4_e4m3_scaled(gb[0], gb[1], gb[2], gb[3], inv1, bnd1), gb[0], gb[1], gb[2], gb[3]);
          uw[k] = fix_nan4(pack4_e4m3_scaled(ub[0], ub[1], ub[2], ub[3], inv1, bnd1), ub[0], ub[1], ub[2], ub[3]);
          hw[k] = fix_nan4(pack4_e4m3_scaled(hb[0], hb[1], hb[2], hb[3], inv2, bnd2), hb[0], hb[1], hb[2], hb[3]);
        }
      }
    }
    store16(Gt + row * kEpiStride + cb, {gw[0], gw[1], gw[2], gw[3]});
    store16(Ut + row * kEpiStride + cb, {uw[0], uw[1], uw[2], uw[3]});
    store16(Ht + row * kEpiStride + cb, {hw[0], hw[1], hw[2], hw[3]});
  }
  m_gu *= deq;
  m_h *= deq * deq;
  __syncthreads();
  // gu8 (gate and up halves) and h8 as 64-column K-slab blocks (every tile
  // row: rows past T are zero padding), then, when asked for, the
  // token-contiguous h8t
  lds_rows_to_kslab<2, 512>(Gt, kTile, kEpiStride, gu8, ldt, m0, n0);
  lds_rows_to_kslab<2, 512>(Ut, kTile, kEpiStride, gu8, ldt, m0, I + n0);
  lds_rows_to_kslab<2, 512>(Ht, kTile, kEpiStride, h8, ldt, m0, n0);
  if (h8t) lds_tile_store_slab_tr<8, 8>(Ht, kEpiStride, h8t, slab_rows(I), m0, n0);
  m_gu = wave_max(m_gu);
  m_h = wave_max(m_h);
  if (lane == 0) { red[wave] = m_gu; red[8 + wave] = m_h; }
  __syncthreads();
  if (tid == 0) {
    float a1 = red[0], a2 = red[8];
#pragma unroll
    for (int w = 1; w < 8; ++w) {
      a1 = fmaxf(a1, red[w]);
      a2 = fmaxf(a2, red[8 + w]);
    }
    atomic_max_nonneg(amax + 1, a1);
    atomic_max_nonneg(amax + 2, a2);
  }
}

// ---------------------------------------------------------------------------
// (a6) gate/up forward + SwiGLU, persistent with a deferred epilogue.
//
// Tile 256 tokens x 64 (gate, up) column pairs: B tile = 64 gate rows + 64 up
// rows (MainLoop NB = 2, paired), so each lane holds g and u of the same 16
// consecutive columns for each of its 4 row blocks.  One work-group per CU
// walks its tiles; after tile i's K loop the lane packs bf16(g), bf16(u) of
// its 64 pairs into 64 registers (E), and the SwiGLU of tile i runs in 16
// units of 4 pairs, one per K stage of tile i+1, in the same instruction
// stream as its MFMAs (the matrix pipe runs them while the vector ALU does the
// epilogue): each unit in six pieces, one after each MFMA past the stage's
// barrier.  The h bytes of a tile also go to one of two LDS
// tiles; its token-contiguous (K-slab) copy is written at the next tile
// boundary with LDS transpose reads.  The last tile's epilogue runs alone.
// NK = D / 64 K stages, fully unrolled so each unit has a fixed stage; the K
// stream runs on across tiles (the last three stages of a tile load the next
// tile's first three), so a tile boundary waits for no DMA.
constexpr int kPipeHStride = 80;                    // 64 h bytes + 16 per LDS row
constexpr int kPipeHBytes = kTile * kPipeHStride;   // one h tile
constexpr int kPipeRing = MainLoop<false, kFmtE4M3, kFmtE4M3, true, 2, 4>::kLds;  // 96 KiB
constexpr int kPipeLds = kPipeRing + 2 * kPipeHBytes + 64;
// the pipe's waves: 8 of 64 x 64 (two row blocks each)
constexpr int kPipeTB = 2;
constexpr int kPipeThreads = kPipeTB == 4 ? 256 : 512;

// B-tile row r of the 128-row paired tile -> (half, column within 64):
// half = r / 64 (gate, up); column = 32*wn + 16*g + v for the lane layout.
SFP8_DEV int paired_col64(int r) {
  const int rl = r & 63, wn = rl >> 5, w = rl & 31;
  return 32 * wn + 16 * ((w >> 2) & 1) + 4 * (w >> 3) + (w & 3);
}

// The h tile's 256 rows of 64 bytes to 256 consecutive K-slab rows (NT
// threads, 16 bytes each per pass).
template <int NT>
SFP8_DEV void pipe_h8_rows(const uint8_t* hbuf, uint8_t* dst) {
#pragma unroll
  for (int k = 0; k < 1024 / NT; ++k) {
    const int idx = NT * k + (int)threadIdx.x, r = idx >> 2, ch = idx & 3;
    *reinterpret_cast<intx4*>(dst + r * 64 + 16 * ch) =
        *reinterpret_cast<const intx4*>(hbuf + r * kPipeHStride + 16 * ch);
  }
}

// TB = row blocks of 32 per wave: 4 (4 waves of 128 x 64) or 2 (8 waves of
// 64 x 64, two per SIMD: each wave's waits are covered by the other's
// MFMAs).
template <int NK, int TB>
struct SwigluPipe {
  using ML = MainLoop<false, kFmtE4M3, kFmtE4M3, true, 2, 4, 0, false, false, 2, TB>;
  static constexpr int kWaves = ML::kWaves, kWM = ML::kWM;
  static constexpr int kUnits = 4 * TB;  // 4 pairs each: unit u = row block u/4, pairs 4*(u%4) ..
  static constexpr int kSt = 4;          // LDS ring stages
  static constexpr int kDma = ML::kDma;
  static constexpr int kPre = TB == 4 ? 2 : 1;  // MFMAs of a stage issued before its wait
  static constexpr int kSpan = NK / kUnits;     // stages per unit
  static constexpr int kSlots = ML::kMfma - kPre;  // MFMAs past the barrier, one slot each
  static constexpr int kDmaSlots = TB == 4 ? 2 : kSlots;  // slots carrying the DMA
  static_assert(NK >= kSt && NK % kSt == 0, "whole rings of K stages: a tile's stage s sits in slot s % kSt");
  static_assert(NK % kUnits == 0 && kSpan * kSlots == 6, "each unit's six pieces fill the slots of its stages");

  // A unit's working values between its pieces.
  struct UnitTmp {
    float gb[4], ub[4], hb[4], ex[4], sg[4];
  };

  struct Ctx {
    // main loop; the last kSt - 1 stages of a tile load the first stages of
    // the next tile (nra, nvoff_b), or repeat this tile's last stage when
    // there is none (has_next false: nra, nvoff_b = ra, voff_b)
    uint8_t* lds;
    __amdgpu_buffer_rsrc_t ra, rb, nra, nrb;
    uint32_t voff_a[4], voff_b[2], nvoff_b[2], aoff[8], boff[8];
    bool has_next;
    int wave;
    typename ML::Frag f[2];
    floatx16 acc[TB][2];
    // previous tile's epilogue
    uint32_t E[TB][16];
    uint32_t gw[4], uw[4], hw[4];
    UnitTmp ut;  // the current unit's working values (its pieces may span two stages)
    bool bad;  // a unit of the current row block saw NaN or out-of-range data
    float m_gu, m_h;
    bool prev;            // a previous tile exists
    int64_t pm0, pn0;     // its origin
    uint8_t* hbuf;        // its LDS h tile
    // scales (of the previous tile's weight: the epilogue's) and outputs
    float deq, c_exp, inv1, bnd1, inv2, bnd2;
    float s0, s1, s2;  // scale[0], scale[1], scale[2]
    float mx_gu, mx_h;  // amax so far, dequantized
    int64_t T, I, ldt;
    // gu8 (the K-slab [2I/64][ldt][64]) and the previous tile's byte offsets
    // in it: gate block (pn0/64, rows pm0..) and up block (I + pn0)/64
    __amdgpu_buffer_rsrc_t rgu;
    uint32_t so_g, so_u;
    uint8_t* h8;
  };

  // One unit: 4 pairs of row block TB, packed into byte Q of gw/uw/hw.
  template <int U>
  static SFP8_DEV void unit_compute(Ctx& c) {
    constexpr int RB = U / 4, Q = U % 4;
    float gb[4], ub[4], hb[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t p = c.E[RB][4 * Q + e];
      gb[e] = __uint_as_float(p << 16);
      ub[e] = __uint_as_float(p & 0xffff0000u);
      const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(gb[e] * c.c_exp));
      hb[e] = gb[e] * sg * ub[e];
    }
    // NaN-propagating maxima of the magnitudes: when both are inside the
    // e4m3 range (after scaling) no clamp can act and no NaN needs patching,
    // so the unclamped conversions are exact; otherwise the row block's
    // block_store redoes them (wave-uniform, rare)
    float a = max3_nan(fabsf(gb[0]), fabsf(ub[0]), fabsf(gb[1]));
    a = max3_nan(a, fabsf(ub[1]), fabsf(gb[2]));
    a = max3_nan(a, fabsf(ub[2]), fabsf(gb[3]));
    a = __builtin_elementwise_maximum(a, fabsf(ub[3]));
    float b = max3_nan(fabsf(hb[0]), fabsf(hb[1]), fabsf(hb[2]));
    b = __builtin_elementwise_maximum(b, fabsf(hb[3]));
    c.bad |= !(a <= c.bnd1) | !(b <= c.bnd2);
    c.m_gu = fmaxf(c.m_gu, a);  // a NaN here is redone by the exact path
    c.m_h = fmaxf(c.m_h, b);
    c.gw[Q] = pack4_e4m3_scaled_noclamp(gb[0], gb[1], gb[2], gb[3], c.inv1, c.gw[Q]);
    c.uw[Q] = pack4_e4m3_scaled_noclamp(ub[0], ub[1], ub[2], ub[3], c.inv1, c.uw[Q]);
    c.hw[Q] = pack4_e4m3_scaled_noclamp(hb[0], hb[1], hb[2], hb[3], c.inv2, c.hw[Q]);
  }

  // Piece P of unit U: the arithmetic of unit_compute<U>, the same
  // operations in the same order per value, cut into six parts that go one
  // after each of the stage's MFMAs past the barrier and software-pipelined
  // over the unit's four pairs (the exponent of a pair one piece before its
  // reciprocal), so that each part holds at most two transcendental
  // instructions (a quarter of the vector ALU's rate) beside independent
  // others.  A wave issues in order: more vector work between two MFMAs
  // than the first one's 64 cycles holds back the second.  Each part reads
  // its inputs and publishes its results through empty asm statements, so
  // the compiler keeps it in its slot.
  template <int RB, int Q, int E>
  static SFP8_DEV void unit_unpack(Ctx& c, UnitTmp& t) {
    uint32_t p = c.E[RB][4 * Q + E];
    asm volatile("" : "+v"(p));
    t.gb[E] = __uint_as_float(p << 16);
    t.ub[E] = __uint_as_float(p & 0xffff0000u);
    t.ex[E] = __builtin_amdgcn_exp2f(t.gb[E] * c.c_exp);
  }
  template <int U, int P>
  static SFP8_DEV void unit_piece(Ctx& c, UnitTmp& t) {
    constexpr int RB = U / 4, Q = U % 4;
    if constexpr (P == 0) {
      unit_unpack<RB, Q, 0>(c, t);
      unit_unpack<RB, Q, 1>(c, t);
      asm volatile("" ::"v"(t.ex[0]), "v"(t.ex[1]));
    } else if constexpr (P == 1) {
      t.sg[0] = __builtin_amdgcn_rcpf(1.0f + t.ex[0]);
      t.sg[1] = __builtin_amdgcn_rcpf(1.0f + t.ex[1]);
      unit_unpack<RB, Q, 2>(c, t);
      asm volatile("" ::"v"(t.sg[0]), "v"(t.sg[1]), "v"(t.ex[2]));
    } else if constexpr (P == 2) {
      unit_unpack<RB, Q, 3>(c, t);
      t.sg[2] = __builtin_amdgcn_rcpf(1.0f + t.ex[2]);
      t.hb[0] = t.gb[0] * t.sg[0] * t.ub[0];
      t.hb[1] = t.gb[1] * t.sg[1] * t.ub[1];
      asm volatile("" ::"v"(t.ex[3]), "v"(t.sg[2]), "v"(t.hb[0]), "v"(t.hb[1]));
    } else if constexpr (P == 3) {
      t.sg[3] = __builtin_amdgcn_rcpf(1.0f + t.ex[3]);
      t.hb[2] = t.gb[2] * t.sg[2] * t.ub[2];
      // NaN-propagating maximum of the gate and up magnitudes: inside the
      // e4m3 range (after scaling) no clamp can act and no NaN needs
      // patching, so the unclamped conversions are exact; otherwise the row
      // block's block_store redoes them (wave-uniform, rare)
      float a = max3_nan(fabsf(t.gb[0]), fabsf(t.ub[0]), fabsf(t.gb[1]));
      a = max3_nan(a, fabsf(t.ub[1]), fabsf(t.gb[2]));
      a = max3_nan(a, fabsf(t.ub[2]), fabsf(t.gb[3]));
      a = __builtin_elementwise_maximum(a, fabsf(t.ub[3]));
      c.bad |= !(a <= c.bnd1);
      c.m_gu = fmaxf(c.m_gu, a);  // a NaN here is redone by the exact path
      asm volatile("" ::"v"(t.sg[3]), "v"(t.hb[2]), "v"(c.m_gu));
    } else if constexpr (P == 4) {
      t.hb[3] = t.gb[3] * t.sg[3] * t.ub[3];
      float b = max3_nan(fabsf(t.hb[0]), fabsf(t.hb[1]), fabsf(t.hb[2]));
      b = __builtin_elementwise_maximum(b, fabsf(t.hb[3]));
      c.bad |= !(b <= c.bnd2);
      c.m_h = fmaxf(c.m_h, b);
      c.gw[Q] = pack4_e4m3_scaled_noclamp(t.gb[0], t.gb[1], t.gb[2], t.gb[3], c.inv1, c.gw[Q]);
      asm volatile("" ::"v"(c.m_h), "v"(c.gw[Q]));
    } else {
      c.uw[Q] = pack4_e4m3_scaled_noclamp(t.ub[0], t.ub[1], t.ub[2], t.ub[3], c.inv1, c.uw[Q]);
      c.hw[Q] = pack4_e4m3_scaled_noclamp(t.hb[0], t.hb[1], t.hb[2], t.hb[3], c.inv2, c.hw[Q]);
      asm volatile("" ::"v"(c.uw[Q]), "v"(c.hw[Q]));
    }
  }

  // After the last unit of row block TB: the exact conversions when a unit
  // of the block saw NaN or out-of-range data (wave-uniform, rare), the
  // three 16-byte global stores and the h bytes into the LDS tile.
  template <int RB>
  static SFP8_DEV void block_store(Ctx& c) {
    const int lane = threadIdx.x & 63, wm = c.wave % kWM, wn = c.wave / kWM;
    const int fr = lane & 31, g = lane >> 5;
    if (__builtin_amdgcn_ballot_w64(c.bad)) {
      asm volatile("" ::: "memory");
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float gb[4], ub[4], hb[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t p = c.E[RB][4 * q + e];
          gb[e] = __uint_as_float(p << 16);
          ub[e] = __uint_as_float(p & 0xffff0000u);
          const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(gb[e] * c.c_exp));
          hb[e] = gb[e] * sg * ub[e];
          // amax over the non-NaN values
          c.m_gu = fmaxf(c.m_gu, fmaxf(fabsf(gb[e]), fabsf(ub[e])));
          c.m_h = fmaxf(c.m_h, fabsf(hb[e]));
        }
        c.gw[q] = fix_nan4(pack4_e4m3_scaled(gb[0], gb[1], gb[2], gb[3], c.inv1, c.bnd1), gb[0], gb[1], gb[2], gb[3]);
        c.uw[q] = fix_nan4(pack4_e4m3_scaled(ub[0], ub[1], ub[2], ub[3], c.inv1, c.bnd1), ub[0], ub[1], ub[2], ub[3]);
        c.hw[q] = fix_nan4(pack4_e4m3_scaled(hb[0], hb[1], hb[2], hb[3], c.inv2, c.bnd2), hb[0], hb[1], hb[2], hb[3]);
      }
    }
    c.bad = false;
    const int row = 32 * TB * wm + 32 * RB + fr;
    const int col = 32 * wn + 16 * g;
    if (c.prev) {
      // gu8 is a K-slab [2I/64][ldt][64], h8 one of [I/64][ldt][64]: the
      // tile's 64 gate, 64 up and 64 h columns are one block each (rows past
      // T hold the zeros computed from x8's zero padding); the block's
      // origin is the store's scalar offset
      const uint32_t vo = (uint32_t)(row * 64 + col);
      __builtin_amdgcn_raw_buffer_store_b128(intx4{(int)c.gw[0], (int)c.gw[1], (int)c.gw[2], (int)c.gw[3]},
                                             c.rgu, vo, (int)c.so_g, 0);
      __builtin_amdgcn_raw_buffer_store_b128(intx4{(int)c.uw[0], (int)c.uw[1], (int)c.uw[2], (int)c.uw[3]},
                                             c.rgu, vo, (int)c.so_u, 0);
    }
    store16(c.hbuf + row * kPipeHStride + col, c.hw);
  }

  // Stage KT: the first kPre MFMAs, then the wait for stage KT+1 and the
  // barrier, then six slots (slot below), then the row-block stores the
  // stage's unit completed.  Vector stores count in vmcnt too and may
  // complete after later loads, so the wait allows only the kDma loads
  // issued after stage KT+1's; stores still in flight can make it wait for
  // those as well.
  template <int KT>
  static SFP8_DEV void stage(Ctx& c, int a_ss, int b_ss) {
    constexpr int cur = KT & 1, nxt = cur ^ 1;
    // the first kPre MFMAs (register operands only) go ahead of the wait,
    // so the matrix core stays busy while it blocks
    ML::template mfma_range<0, kPre>(c.f[cur], c.acc);
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kDma * (kSt - 3)) : "memory");
    __builtin_amdgcn_sched_barrier(0);
    slots<KT, 0>(c, c.ut, a_ss, b_ss);
    // the stage that finishes a unit that finishes a row block stores it
    constexpr int U = KT / kSpan;
    if constexpr (KT % kSpan == kSpan - 1 && U % 4 == 3) block_store<U / 4>(c);
  }
  template <int KT, int J>
  static SFP8_DEV void slots(Ctx& c, UnitTmp& t, int a_ss, int b_ss) {
    if constexpr (J < kSlots) {
      slot<KT, J>(c, t, a_ss, b_ss);
      slots<KT, J + 1>(c, t, a_ss, b_ss);
    }
  }

  // Slot J of stage KT: one MFMA past the barrier, then (J < 2) half of the
  // DMA of stage KT+3 (of the next tile past the last stage), one fragment
  // of stage KT+1 (B blocks first: the next stage's first MFMAs use b[0],
  // b[1] and a[0]) and piece J of the stage's epilogue unit; the scheduling
  // barrier keeps the slot's work after its MFMA.
  template <int KT, int J>
  static SFP8_DEV void slot(Ctx& c, UnitTmp& t, int a_ss, int b_ss) {
    constexpr int cur = KT & 1, nxt = cur ^ 1;
    ML::template mfma_range<kPre + J, kPre + J + 1>(c.f[cur], c.acc);
    if constexpr (J < kDmaSlots) {
      constexpr int slot_ = (KT + kSt - 1) % kSt;
#pragma unroll
      for (int j = J * kDma / kDmaSlots; j < (J + 1) * kDma / kDmaSlots; ++j) {
        if constexpr (KT + kSt - 1 < NK) {
          constexpr int ld = KT + kSt - 1;
          ML::load_one(j, c.lds, slot_, c.ra, c.rb, c.voff_a, c.voff_b, stage_off<ld>(a_ss), stage_off<ld>(b_ss),
                       c.wave);
        } else {
          const int ld = c.has_next ? KT + kSt - 1 - NK : NK - 1;
          ML::load_one(j, c.lds, slot_, c.nra, c.nrb, c.voff_a, c.nvoff_b, ld * a_ss, ld * b_ss, c.wave);
        }
      }
    }
    if constexpr (TB == 4) {
      ML::template read_frag<J < 2 ? 4 + J : J - 2>(c.lds, (KT + 1) % kSt, c.aoff, c.boff, c.f[nxt]);
    } else if constexpr (J == 0) {
      // a[0] and b[0] first (the next stage's MFMA ahead of its wait), then
      // b[1], then a[1]
      ML::template read_frag<0>(c.lds, (KT + 1) % kSt, c.aoff, c.boff, c.f[nxt]);
      ML::template read_frag<2>(c.lds, (KT + 1) % kSt, c.aoff, c.boff, c.f[nxt]);
    } else {
      ML::template read_frag<J == 1 ? 3 : 1>(c.lds, (KT + 1) % kSt, c.aoff, c.boff, c.f[nxt]);
    }
    unit_piece<KT / kSpan, (KT % kSpan) * kSlots + J>(c, t);
    __builtin_amdgcn_sched_barrier(0);
  }

  // Stage LD's byte offset LD * ss, computed where it is used (otherwise
  // the products for all fixed stages stay live in scalar registers across
  // the tile loop).
  template <int LD>
  static SFP8_DEV int stage_off(int ss) {
    asm volatile("" : "+s"(ss));
    return LD * ss;
  }

  template <int KT>
  static SFP8_DEV void stages(Ctx& c, int a_ss, int b_ss) {
    if constexpr (KT < NK) {
      stage<KT>(c, a_ss, b_ss);
      stages<KT + 1>(c, a_ss, b_ss);
    }
  }
  template <int U0>
  static SFP8_DEV void tail_units(Ctx& c) {
    if constexpr (U0 < kUnits) {
      unit_compute<U0>(c);
      if constexpr (U0 % 4 == 3) block_store<U0 / 4>(c);
      tail_units<U0 + 1>(c);
    }
  }

  // The finished epilogue's maxima, dequantized with its tile's scale, join
  // the running amax (exact: the scales are powers of two); then the next
  // epilogue's constants for weight scale q (all powers of two).
  static SFP8_DEV void next_scales(Ctx& c, float q) {
    c.mx_gu = fmaxf(c.mx_gu, c.m_gu * c.deq);
    c.mx_h = fmaxf(c.mx_h, c.m_h * (c.deq * c.deq));
    c.m_gu = 0.f;
    c.m_h = 0.f;
    c.deq = 1.0f / (c.s0 * q);
    c.c_exp = c.deq * -1.4426950408889634f;
    const float m1 = c.deq * c.s1, m2 = c.deq * c.deq * c.s2;
    c.inv1 = 1.0f / m1;
    c.inv2 = 1.0f / m2;
    c.bnd1 = kE4M3Max * c.inv1;
    c.bnd2 = kE4M3Max * c.inv2;
  }
};

template <int NK, int TB>
__global__ __launch_bounds__(TB == 4 ? 256 : 512, 1) void swiglu_pipe_kernel(
    const uint8_t* __restrict__ x8, const uint8_t* __restrict__ w8, int64_t T, int64_t D, int64_t I,
    const float* __restrict__ scale, const float* __restrict__ wscale, float* __restrict__ amax,
    uint8_t* __restrict__ gu8, uint8_t* __restrict__ h8, uint8_t* __restrict__ h8t, int64_t ldt, int tiles_m,
    int tiles_n, const int* __restrict__ plan, int64_t w_estride) {
  using P = SwigluPipe<NK, TB>;
  using ML = typename P::ML;
  extern __shared__ __align__(16) uint8_t lds[];
  typename P::Ctx c;
  c.lds = lds;
  c.wave = threadIdx.x >> 6;
  // scales folded as in swiglu_fwd_kernel (all powers of two); with a plan
  // each tile's expert has its own weight scale wscale[e]
  c.s0 = scale[0];
  c.s1 = scale[1];
  c.s2 = scale[2];
  c.m_gu = 0.f;
  c.m_h = 0.f;
  c.mx_gu = 0.f;
  c.mx_h = 0.f;
  c.deq = 1.f;
  P::next_scales(c, wscale[0]);
  if (plan) tiles_m = MoePlan{plan}.ntiles();
  c.T = T;
  c.I = I;
  c.ldt = ldt;
  c.rgu = make_rsrc(gu8, 2 * I * ldt);
  c.so_g = c.so_u = 0u;
  c.h8 = h8;
  c.bad = false;
#pragma unroll
  for (int q = 0; q < 4; ++q) c.gw[q] = c.uw[q] = c.hw[q] = 0u;
  c.prev = false;
  c.pm0 = 0;
  c.pn0 = 0;
  c.hbuf = lds + kPipeRing;
  // the first tile's K loop runs the epilogue units with no previous tile:
  // on zeros they add nothing to the amax slots (and store nothing)
#pragma unroll
  for (int tb = 0; tb < TB; ++tb)
#pragma unroll
    for (int v = 0; v < 16; ++v) c.E[tb][v] = 0u;
  const int lane = threadIdx.x & 63, wm = c.wave % P::kWM, wn = c.wave / P::kWM;
  const int fr = lane & 31, g = lane >> 5;
  const uint32_t chunk = (uint32_t)(((lane & 3) ^ ((lane >> 4) & 3)) << 4);
  const int sw = (fr >> 2) & 3;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    c.aoff[h] = (uint32_t)((32 * TB * wm + fr) * kStage + (((2 * g + h) ^ sw) << 4));
    c.boff[h] = (uint32_t)(ML::kLdsB + (BLayout<true, 2>::kWaveStride * wn + fr) * kStage + (((2 * g + h) ^ sw) << 4));
  }
  const int64_t rpad = slab_rows(I);
  const int ntiles = tiles_m * tiles_n;
  const int a_ss = (int)(ldt * kStage), b_ss = (int)(2 * I * kStage);
#pragma unroll
  for (int j = 0; j < ML::kDmaA; ++j)
    c.voff_a[j] = (uint32_t)(((kTile / P::kWaves) * c.wave + 16 * j + (lane >> 2)) * kStage) + chunk;
  // K-slab operands: x8 [D/64][ldt][64], w8 [D/64][2I][64] (with a plan:
  // tile row tm's expert e at w8 + e * w_estride, its scale wscale[e]); tile
  // origin (m0, n0) -> A and B descriptors, B lane offsets, weight scale
  auto tile_operands = [&](int tile, int64_t& m0, int64_t& n0, __amdgpu_buffer_rsrc_t& ra,
                           __amdgpu_buffer_rsrc_t& rb, uint32_t (&voff_b)[2], float& q) {
    int tm, tn;
    tile_coords(tile, ntiles, tiles_m, tiles_n, tm, tn);
    m0 = (int64_t)tm * kTile;
    n0 = (int64_t)tn * 64;
    ra = make_rsrc(x8 + m0 * kStage, D * ldt - m0 * kStage);
    const int e = plan ? MoePlan{plan}.expert(tm) : 0;
    rb = make_rsrc(w8 + e * w_estride, D * 2 * I);
    q = wscale[e];
#pragma unroll
    for (int j = 0; j < ML::kDmaB; ++j) {
      const int r = (128 / P::kWaves) * c.wave + 16 * j + (lane >> 2);
      voff_b[j] = (uint32_t)(((r >> 6) * (int)I + (int)n0 + paired_col64(r)) * kStage) + chunk;
    }
  };
  int it = 0;
  int64_t m0 = 0, n0 = 0;
  float q = 1.f, nq = 1.f;  // weight scale of the current tile and of the next
  if (blockIdx.x < ntiles) {
    // prologue, once per work-group: the first tile's stages 0..2 in flight,
    // stage 0 landed, its fragments read.  Later tiles' first stages are
    // loaded by the last stages of the tile before.
    tile_operands(blockIdx.x, m0, n0, c.ra, c.rb, c.voff_b, q);
#pragma unroll
    for (int s = 0; s < 3; ++s) ML::load_stage(lds, s, c.ra, c.rb, c.voff_a, c.voff_b, s * a_ss, s * b_ss, c.wave);
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(2 * ML::kDma) : "memory");
    ML::read_frags(lds, 0, c.aoff, c.boff, c.f[0]);
  }
  for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x, ++it) {
    int64_t nm0 = m0, nn0 = n0;
    c.has_next = tile + (int)gridDim.x < ntiles;
    if (c.has_next) {
      tile_operands(tile + (int)gridDim.x, nm0, nn0, c.nra, c.nrb, c.nvoff_b, nq);
    } else {
      c.nra = c.ra;
      c.nrb = c.rb;
      c.nvoff_b[0] = c.voff_b[0];
      c.nvoff_b[1] = c.voff_b[1];
    }
#pragma unroll
    for (int i = 0; i < TB; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) c.acc[i][j] = floatx16{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f,
                                                          0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    P::template stages<0>(c, a_ss, b_ss);
    // every wave's h-tile writes are done (the next tile's first stages stay
    // in flight)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // the previous tile's h tile is complete: its K-slab copies (h8: 256
    // token rows of 64 bytes, one contiguous block; the optional h8t
    // transposed)
    if (c.prev) {
      pipe_h8_rows<64 * P::kWaves>(c.hbuf, h8 + (c.pn0 >> 6) * ldt * 64 + c.pm0 * 64);
      if (h8t) lds_tile_store_slab_tr<4, P::kWaves>(c.hbuf, kPipeHStride, h8t, rpad, c.pm0, c.pn0);
    }
    // this tile's g, u (bf16, unscaled) become the next epilogue's input
#pragma unroll
    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
      for (int v = 0; v < 16; ++v) c.E[tb][v] = pack2_bf16(c.acc[tb][0][v], c.acc[tb][1][v]);
    c.prev = true;
    c.pm0 = m0;
    c.pn0 = n0;
    c.so_g = (uint32_t)((n0 >> 6) * ldt * 64 + m0 * 64);
    c.so_u = (uint32_t)(((I + n0) >> 6) * ldt * 64 + m0 * 64);
    c.hbuf = lds + kPipeRing + (it & 1) * kPipeHBytes;
    // the previous epilogue is complete: its amax joins, and this tile's
    // weight scale sets the next epilogue's constants
    P::next_scales(c, q);
    m0 = nm0;
    n0 = nn0;
    q = nq;
    c.ra = c.nra;
    c.rb = c.nrb;
    c.voff_b[0] = c.nvoff_b[0];
    c.voff_b[1] = c.nvoff_b[1];
  }
  // the last tile's repeated loads of its last stage are still in flight
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if (c.prev) {
    P::template tail_units<0>(c);
    __syncthreads();
    pipe_h8_rows<64 * P::kWaves>(c.hbuf, h8 + (c.pn0 >> 6) * ldt * 64 + c.pm0 * 64);
    if (h8t) lds_tile_store_slab_tr<4, P::kWaves>(c.hbuf, kPipeHStride, h8t, rpad, c.pm0, c.pn0);
  }
  P::next_scales(c, 1.f);  // folds the last epilogue's maxima
  float* red = reinterpret_cast<float*>(lds + kPipeRing + 2 * kPipeHBytes);
  float mg = wave_max(c.mx_gu), mh = wave_max(c.mx_h);
  if (lane == 0) {
    red[c.wave] = mg;
    red[P::kWaves + c.wave] = mh;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float a1 = red[0], a2 = red[P::kWaves];
#pragma unroll
    for (int w = 1; w < P::kWaves; ++w) {
      a1 = fmaxf(a1, red[w]);
      a2 = fmaxf(a2, red[P::kWaves + w]);
    }
    atomic_max_nonneg(amax + 1, a1);
    atomic_max_nonneg(amax + 2, a2);
  }
}

// bf16 epilogues stage the tile in two passes of 128 rows (256 bf16 columns,
// row stride kBf16Stride: consecutive rows shift by 4 banks) and then write
// whole rows.  Pass P holds tile rows 64P..64P+63 and 128+64P..128+64P+63.
constexpr int kBf16Stride = 528;

template <int P>
SFP8_DEV void stage_bf16_half(uint8_t* lds, const floatx16 (&acc)[4][4], float s) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, wm = wave & 1, wn = wave >> 1;
  const int fr = lane & 31, g = lane >> 5, cb = 128 * wn + 64 * g;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int lr = 64 * wm + 32 * tt + fr;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      uint32_t w0[4], w1[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        w0[i] = pack2_bf16(acc[2 * P + tt][nb][2 * i] * s, acc[2 * P + tt][nb][2 * i + 1] * s);
        w1[i] = pack2_bf16(acc[2 * P + tt][nb][8 + 2 * i] * s, acc[2 * P + tt][nb][8 + 2 * i + 1] * s);
      }
      uint8_t* q = lds + lr * kBf16Stride + (cb + 16 * nb) * 2;
      store16(q, w0);
      store16(q + 16, w1);
    }
  }
}

// The same for the 8-wave tile layout (wave (wm, wn), wn = 0..3, owns A rows
// 128 wm.. and output columns 64 wn.. as 4 x 2 blocks; lane half g of block
// nb holds columns 64 wn + 32 g + 16 nb + v).
template <int P>
SFP8_DEV void stage_bf16_half8(uint8_t* lds, const floatx16 (&acc)[4][2], float s) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, wm = wave & 1, wn = wave >> 1;
  const int fr = lane & 31, g = lane >> 5, cb = 64 * wn + 32 * g;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int lr = 64 * wm + 32 * tt + fr;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      uint32_t w0[4], w1[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        w0[i] = pack2_bf16(acc[2 * P + tt][nb][2 * i] * s, acc[2 * P + tt][nb][2 * i + 1] * s);
        w1[i] = pack2_bf16(acc[2 * P + tt][nb][8 + 2 * i] * s, acc[2 * P + tt][nb][8 + 2 * i + 1] * s);
      }
      uint8_t* q = lds + lr * kBf16Stride + (cb + 16 * nb) * 2;
      store16(q, w0);
      store16(q + 16, w1);
    }
  }
}

// Tile row held in staging row lr of pass p.
SFP8_DEV int half_tile_row(int lr, int p) { return 128 * (lr >> 6) + 64 * p + (lr & 63); }

// Byte offset of out[t, n] (bf16, leading dimension ld) from out + m0 * ld,
// or 2^31 -- past the range of any descriptor, so the store is dropped --
// for t >= T or n >= N.  A bit mask rather than a select keeps the stores
// free of branches (one store instruction per chunk, a fixed count per
// wave).  Tile rows t - m0 < 256, so the offset needs ld < 2^22.
SFP8_DEV uint32_t bf16_out_off(int64_t t, int64_t n, int64_t m0, int64_t T, int64_t N, int64_t ld) {
  const uint32_t in = 0u - (uint32_t)(t < T && n < N);
  return ((uint32_t)(((t - m0) * ld + n) * 2) & in) | (~in & 0x80000000u);
}

// Writes one staged pass to out[t, n] (bf16, leading dimension ld) for rows
// m0.. of the tile below T and columns below N.  NT = threads of the
// work-group.
template <int NT = 256>
SFP8_DEV void write_bf16_half(const uint8_t* lds, int p, int64_t m0, int64_t n0, int64_t T, int64_t N,
                              int64_t ld, uint16_t* __restrict__ out) {
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(out + m0 * ld, (T - m0) * ld * 2);
#pragma unroll
  for (int k = 0; k < 4096 / NT; ++k) {
    const int idx = (int)threadIdx.x + NT * k;
    const int lr = idx >> 5, c = idx & 31;
    const int64_t t = m0 + half_tile_row(lr, p), n = n0 + 8 * c;
    const intx4 o = *reinterpret_cast<const intx4*>(lds + lr * kBf16Stride + c * 16);
    __builtin_amdgcn_raw_buffer_store_b128(o, ro, bf16_out_off(t, n, m0, T, N, ld), 0, 0);
  }
}

// Residual words of staged half p, in write_bf16_half's order (4096 / NT per
// thread); rows past T read as zero through the descriptor.
template <int NT>
SFP8_DEV void load_res_half(__amdgpu_buffer_rsrc_t rres, int p, int64_t n0, int64_t D, intx4 (&rv)[4096 / NT]) {
#pragma unroll
  for (int k = 0; k < 4096 / NT; ++k) {
    const int idx = (int)threadIdx.x + NT * k;
    const int lr = idx >> 5, c = idx & 31;
    const uint32_t off = (uint32_t)((half_tile_row(lr, p) * D + n0 + 8 * c) * 2);
    rv[k] = __builtin_amdgcn_raw_buffer_load_b128(rres, off, 0, kNT);
  }
}

// write_bf16_half after adding the bf16 residual, already in registers:
// out = bf16(res + staged).
template <int NT>
SFP8_DEV void write_bf16_half_res(const uint8_t* lds, int p, int64_t m0, int64_t n0, int64_t T, int64_t D,
                                  const intx4 (&rv)[4096 / NT], uint16_t* __restrict__ out) {
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(out + m0 * D, (T - m0) * D * 2);
#pragma unroll
  for (int k = 0; k < 4096 / NT; ++k) {
    const int idx = (int)threadIdx.x + NT * k;
    const int lr = idx >> 5, c = idx & 31;
    const int64_t t = m0 + half_tile_row(lr, p), n = n0 + 8 * c;
    intx4 o = *reinterpret_cast<const intx4*>(lds + lr * kBf16Stride + c * 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t a = (uint32_t)rv[k][i], b = (uint32_t)o[i];
      o[i] = (int)pack2_bf16(__uint_as_float(b << 16) + __uint_as_float(a << 16),
                             __uint_as_float(b & 0xffff0000u) + __uint_as_float(a & 0xffff0000u));
    }
    __builtin_amdgcn_raw_buffer_store_b128(o, ro, bf16_out_off(t, n, m0, T, D, D), 0, 0);
  }
}

// ---------------------------------------------------------------------------
// (a7) down forward + residual (spark-gpt train.py:1019-1046):
//   y = bf16(res + bf16(acc / (s2 * q_d)))
// With a MoE plan: no residual; tile row tm of padded expert order writes
// its rows(tm) valid rows to y rows urow(tm).. (expert order, unpadded);
// W_down8 of expert e at wd8 + e * w_estride, its scale wscale[e] (the dense
// call passes wscale + 1: [q_gu, q_d]).
__global__ __launch_bounds__(512, 1) void down_fwd_kernel(
    const uint8_t* __restrict__ h8, const uint8_t* __restrict__ wd8, const uint16_t* __restrict__ res,
    int64_t T, int64_t D, int64_t I, const float* __restrict__ scale, const float* __restrict__ wscale,
    uint16_t* __restrict__ y, int64_t ldt, int tiles_m, int tiles_n, const int* __restrict__ plan,
    int64_t w_estride) {
  extern __shared__ __align__(16) uint8_t lds[];
  int tm, tn;
  tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
  int64_t u0 = 0, urows = 0;
  if (plan) {
    const MoePlan P{plan};
    if (tm >= P.ntiles()) return;  // work-group uniform
    const int e = P.expert(tm);
    wd8 += e * w_estride;
    wscale += e;
    u0 = P.urow(tm);
    urows = P.rows(tm);
  }
  const int64_t m0 = (int64_t)tm * kTile, n0 = (int64_t)tn * kTile;
  floatx16 acc[4][2];
  // K-slab operands: h8 [I/64][ldt][64], wd8 [I/64][slab_rows(D)][64]
  const int64_t dp = slab_rows(D);
  MainLoop<false, kFmtE4M3, kFmtE4M3, false, 2, kStages, 0, false, false, 4>::run(
      lds, h8 + m0 * kStage, I * ldt - m0 * kStage, [=](int r) { return r * kStage; }, (int)(ldt * kStage),
      wd8 + n0 * kStage, I * dp - n0 * kStage, [=](int r) { return plain_col_nb<2>(r) * kStage; },
      (int)(dp * kStage), (int)(I / kStage), acc);
  const float deq = 1.0f / (scale[2] * wscale[0]);
  if (plan) {
    // expert rows, no residual: out rounded to bf16 (train.py:1377-1378 stores acc / (s2 q_d) as bf16)
    stage_bf16_half8<0>(lds, acc, deq);
    __syncthreads();
    write_bf16_half<512>(lds, 0, u0, n0, u0 + urows, D, D, y);
    __syncthreads();
    stage_bf16_half8<1>(lds, acc, deq);
    __syncthreads();
    write_bf16_half<512>(lds, 1, u0, n0, u0 + urows, D, D, y);
    return;
  }
  const __amdgpu_buffer_rsrc_t rres = make_rsrc(res + m0 * D, (T - m0) * D * 2);
  // Every residual word the two staged halves add is requested at once (one
  // memory latency), in the order the staged rows are written, so both the
  // residual reads and the y writes are whole rows; rows past T read as zero
  // through the descriptor's range check and are not stored.
  intx4 rv0[8], rv1[8];
  load_res_half<512>(rres, 0, n0, D, rv0);
  load_res_half<512>(rres, 1, n0, D, rv1);
  // out rounded to bf16 before the residual add (train.py:1043)
  stage_bf16_half8<0>(lds, acc, deq);
  __syncthreads();
  write_bf16_half_res<512>(lds, 0, m0, n0, T, D, rv0, y);
  __syncthreads();
  stage_bf16_half8<1>(lds, acc, deq);
  __syncthreads();
  write_bf16_half_res<512>(lds, 1, m0, n0, T, D, rv1, y);
}

// ---------------------------------------------------------------------------
// (a9) bf16 down dgrad + SwiGLU backward (spark-gpt train.py:1049-1094):
//   dh = bf16(dy @ Wd); g, u = gu8 / s1; sig = sigmoid(g)
//   d_gate = dh*u*(sig*(1+g*(1-sig))), d_up = dh*g*sig
//   dgu8 = e5m2(d * s3) as the K-slab of [T, 2I] (and optionally of [2I,
//   ldt]: the token-contiguous dgu8t), amax slot 3.
// B = Wd^T (bf16, [I, D]).  Tile 256 tokens x 256 intermediate columns,
// one work-group of 8 waves (two per SIMD, each 128 x 64 of the tile): the
// second wave on a SIMD runs while the first waits, in the K loop and above
// all in the epilogue, whose loads, LDS round trips and barriers a single
// wave per SIMD left exposed.
constexpr int kEpiStride2 = 272;
// LDS: the SwiGLU backward's table at offset 0 (so that an entry's address
// is its code times 8), then the main loop's ring, later the epilogue's
// staging tiles and 8 reduction slots
constexpr int kDgradLutBytes = 256 * 8;

// dg, du of the 4 columns of group w of a 16-column chunk: dh from the
// staged bf16 words h0 (columns 0-7) and h1 (8-15), the gate and up codes
// from gw and uw, the two factors per gate code from the table at LDS
// address 0 (entry b at 8 b: the kernel has no static LDS, so its dynamic
// LDS begins at 0, and one shift of the selected byte is the address); the
// reference's order (train.py:1083-1087).
typedef __attribute__((address_space(3))) const floatx2* lds_floatx2_ptr;
SFP8_DEV void dgrad_swiglu4(const intx4& h0, const intx4& h1, uint32_t gw, uint32_t uw, int w, float (&dg)[4],
                            float (&du)[4]) {
  const uint32_t hw0 = (uint32_t)(w < 2 ? h0[2 * w] : h1[2 * w - 4]);
  const uint32_t hw1 = (uint32_t)(w < 2 ? h0[2 * w + 1] : h1[2 * w - 3]);
  const float dhv[4] = {__uint_as_float(hw0 << 16), __uint_as_float(hw0 & 0xffff0000u), __uint_as_float(hw1 << 16),
                        __uint_as_float(hw1 & 0xffff0000u)};
  const floatx2 g01 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(gw, 1.0f, false);
  const floatx2 g23 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(gw, 1.0f, true);
  const floatx2 u01 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(uw, 1.0f, false);
  const floatx2 u23 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(uw, 1.0f, true);
  const float g8v[4] = {g01.x, g01.y, g23.x, g23.y}, u8v[4] = {u01.x, u01.y, u23.x, u23.y};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    // (sig, sig * (1 + g * (1 - sig)))
    const floatx2 f = *reinterpret_cast<lds_floatx2_ptr>((uintptr_t)(((gw >> (8 * e)) & 0xFFu) << 3));
    dg[e] = (dhv[e] * u8v[e]) * f.y;
    du[e] = (dhv[e] * g8v[e]) * f.x;
  }
}

// With a MoE plan: tile rows are padded expert order (gu8, dgu8, dgu8t over
// ldt padded rows); dy is the row-major upstream gradient of the expert-order
// rows (its rows urow(tm).. for tile row tm), W_down^T of expert e at
// wdt + e * w_estride (bytes); the tile count comes from the plan.
// TCOPY: dgu8t is written too (staged in LDS per pass).
template <bool TCOPY>
__global__ __launch_bounds__(512, 1) void down_dgrad_swiglu_kernel(
    const uint16_t* __restrict__ dy, const uint16_t* __restrict__ wdt, const uint8_t* __restrict__ gu8,
    int64_t T, int64_t D, int64_t I, const float* __restrict__ scale, float* __restrict__ amax,
    uint8_t* __restrict__ dgu8, uint8_t* __restrict__ dgu8t, int64_t ldt, int tiles_m, int tiles_n,
    const int* __restrict__ plan, int64_t w_estride) {
  using Loop = MainLoop<true, 0, 0, false, 2, kStages, 0, false, false, 4>;
  extern __shared__ __align__(16) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t ldb = D * 2;  // bytes
  const int64_t ip = slab_rows(I);
  // The gate operand of the SwiGLU backward is an e4m3 code here, so its two
  // factors take 256 values per launch: entry b of this table holds
  //   sig = sigmoid(g), sig * (1 + g * (1 - sig))   for g = e4m3(b) / s1,
  // rounded in the reference's order (train.py:1083-1087, no contraction).
  // Its LDS range is disjoint from the main loop's ring and the staging
  // tiles; the main loop's first barrier publishes it.
  floatx2* lut = reinterpret_cast<floatx2*>(lds);
  uint8_t* const base = lds + kDgradLutBytes;  // the ring and the staging tiles
  if (tid < 256) {
#pragma clang fp contract(off)
    const float gl = __builtin_amdgcn_cvt_f32_fp8(tid, 0) * (1.0f / scale[1]);
    const float sig = 1.0f / (1.0f + expf(-gl));
    lut[tid] = floatx2{sig, sig * (1.0f + gl * (1.0f - sig))};
  }
  // g = g8*s_gu, u = u8*s_gu with g8, u8 the stored e4m3 values; as the scales
  // are powers of two, d_gate = dg*s_gu and d_up = du*s_gu with
  //   dg = (dh*u8)*(sig*(1 + g*(1-sig))),  du = (dh*g8)*sig  (factors from lut),
  //   dgu8 = e5m2(d*q3) = e5m2(d'*(s_gu*q3)),  amax3 = s_gu*max(|dg|,|du|).
  const float m3s = (1.0f / scale[1]) * scale[3];
  const float inv3 = 1.0f / m3s, bnd3 = kE5M2Max * inv3;
  float* red = reinterpret_cast<float*>(base + 2 * kTile * kEpiStride2);  // 8 floats after the staging tiles
  float m3 = 0.f;
  // Persistent: work-group pid runs tiles pid, pid + gridDim.x, ...  (Work-
  // groups started a quarter of a tile apart per XCD, so that the tiles'
  // 256 KiB store bursts would not coincide, measured 2 % slower.)
  if (plan) tiles_m = MoePlan{plan}.ntiles();
  const int ntiles = tiles_m * tiles_n;
  // A = dy row-major (rows past the tile's last read as zero through the
  // range check); B = Wd^T as a bf16 K-slab [2D/64][slab_rows(I)][64] (bytes)
  const auto arow = [=](int r) { return r * (int)ldb; };
  const auto brow = [=](int r) { return plain_col_nb<2>(r) * kStage; };
  const int nk = (int)(ldb / kStage);
  // the operands of tile `tile`: dy rows m0.. (dense) or the expert rows
  // urow(tm).. (MoE), and W_down^T (of the tile's expert) from column n0
  struct Ops {
    const uint8_t* a;
    int64_t a_bytes;
    const uint8_t* b;
    int64_t b_bytes;
  };
  const auto ops_of = [=](int tm, int tn) {
    const int64_t m0 = (int64_t)tm * kTile, n0 = (int64_t)tn * kTile;
    int64_t a_row = m0, a_rows = T - m0;
    const uint8_t* wb = reinterpret_cast<const uint8_t*>(wdt);
    if (plan) {
      const MoePlan P{plan};
      a_row = P.urow(tm);
      a_rows = P.rows(tm);
      wb += P.expert(tm) * w_estride;
    }
    return Ops{reinterpret_cast<const uint8_t*>(dy) + a_row * ldb, a_rows * ldb, wb + n0 * kStage,
               ldb * ip - n0 * kStage};
  };
  for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
  int tm, tn;
  tile_coords(tile, ntiles, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * kTile, n0 = (int64_t)tn * kTile;
  floatx16 acc[4][2];
  {
    const Ops o = ops_of(tm, tn);
    Loop::run(base, o.a, o.a_bytes, arow, kStage, o.b, o.b_bytes, brow, (int)(ip * kStage), nk, acc);
  }
  // Row-order epilogue, in two passes of 128 tile rows (the rows of
  // stage_bf16_half<P>): dh staged in LDS as bf16, then each thread takes
  // 16-column chunks of one row, reading gu8 and writing dgu8 as whole K-slab
  // rows; with dgu8t the codes also go to LDS for the token-contiguous copy.
  const __amdgpu_buffer_rsrc_t rgu = make_rsrc(gu8 + m0 * 64, 2 * I * ldt - m0 * 64);
  const int cols = (int)((I - n0) < kTile ? (I - n0) : kTile);  // 128 or 256
  uint8_t* DH = base;
  // the staging tiles of the token-contiguous copy (MoE only); their offset
  // goes through an empty asm so that the compiler does not hoist per-lane
  // addresses into them out of the tile loop (a register it had to spill)
  int g2off = kDgradLutBytes + 128 * kBf16Stride;
  asm volatile("" : "+s"(g2off));
  uint8_t* G2 = lds + g2off;
  uint8_t* U2 = G2 + 128 * kEpiStride2;
  // Byte offset from gu8 / dgu8 + m0 * 64 of tile row `row`, tile column c
  // of the gate half (the up half lies I * ldt further, and I * ldt < 2^31):
  // a column past I gets offset 2^31, beyond the descriptors' range in both
  // halves, so its loads return zero and its stores are dropped -- every
  // chunk issues its instructions, a fixed count per wave, with no branch
  // around them (a bit mask rather than a select, which the compiler turned
  // into one).
  const auto gu_off = [=](int c, int row) {
    const int64_t j = n0 + c;
    const uint32_t in = 0u - (uint32_t)(j < I);  // all ones for a column inside I
    return ((uint32_t)((j >> 6) * ldt * 64 + row * 64 + (j & 63)) & in) | (~in & 0x80000000u);
  };
  const __amdgpu_buffer_rsrc_t rdg = make_rsrc(dgu8 + m0 * 64, 2 * I * ldt - m0 * 64);
  // gu8 words of this thread's 4 chunks of pass P, requested at once
  intx4 wg[4], wu[4];
  const auto gu_loads = [&](int P) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int item = 8 * k + wave, slab = item & 3, lr = 16 * (item >> 2) + (lane >> 2);
      const int c = 64 * slab + 16 * (lane & 3);
      const int row = half_tile_row(lr, P);
      wg[k] = __builtin_amdgcn_raw_buffer_load_b128(rgu, gu_off(c, row), 0, kNT);
      wu[k] = __builtin_amdgcn_raw_buffer_load_b128(rgu, gu_off(c, row) + (uint32_t)(I * ldt), 0, kNT);
    }
  };
  // the codes of chunk k of pass P (dh from the staged tile, gate and up
  // codes from wg[k], wu[k]); the running amax in m3
  const auto swiglu_chunk = [&](int P, int k, uint32_t (&pg)[4], uint32_t (&pu)[4]) {
    const int item = 8 * k + wave, slab = item & 3, lr = 16 * (item >> 2) + (lane >> 2);
    const int c = 64 * slab + 16 * (lane & 3);
    const intx4 h0 = *reinterpret_cast<const intx4*>(DH + lr * kBf16Stride + 2 * c);
    const intx4 h1 = *reinterpret_cast<const intx4*>(DH + lr * kBf16Stride + 2 * c + 16);
    // The 16 values' unclamped codes and their NaN-propagating maximum
    // magnitude (the first maximum3 of each group of four takes the
    // running maximum): when it is inside the e5m2 range (after scaling)
    // no clamp can act and no NaN needs its code, so the codes are
    // exact; otherwise (wave-uniform, NaN or out-of-range data only) the
    // chunk is computed again with the clamps and NaN codes, and the amax
    // over its non-NaN values.
    float mc = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      float dg[4], du[4];
      dgrad_swiglu4(h0, h1, (uint32_t)wg[k][w], (uint32_t)wu[k][w], w, dg, du);
      mc = max3_nan(mc, fabsf(dg[0]), fabsf(du[0]));
      mc = max3_nan(mc, fabsf(dg[1]), fabsf(du[1]));
      mc = max3_nan(mc, fabsf(dg[2]), fabsf(du[2]));
      mc = max3_nan(mc, fabsf(dg[3]), fabsf(du[3]));
      // the unclamped packs overwrite both halves of their third argument:
      // the dead dh words, rather than a copy of a live register
      pg[w] = pack4_e5m2_scaled_noclamp(dg[0], dg[1], dg[2], dg[3], inv3,
                                        (uint32_t)(w < 2 ? h0[2 * w] : h1[2 * w - 4]));
      pu[w] = pack4_e5m2_scaled_noclamp(du[0], du[1], du[2], du[3], inv3,
                                        (uint32_t)(w < 2 ? h0[2 * w + 1] : h1[2 * w - 3]));
    }
    if (__builtin_amdgcn_ballot_w64(!(mc <= bnd3))) {
      asm volatile("" ::: "memory");
      mc = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        float dg[4], du[4];
        dgrad_swiglu4(h0, h1, (uint32_t)wg[k][w], (uint32_t)wu[k][w], w, dg, du);
        pg[w] = fix_nan4(pack4_e5m2_scaled(dg[0], dg[1], dg[2], dg[3], inv3, bnd3), dg[0], dg[1], dg[2], dg[3]);
        pu[w] = fix_nan4(pack4_e5m2_scaled(du[0], du[1], du[2], du[3], inv3, bnd3), du[0], du[1], du[2], du[3]);
#pragma unroll
        for (int e = 0; e < 4; ++e) mc = fmaxf(mc, fmaxf(fabsf(dg[e]), fabsf(du[e])));
      }
    }
    m3 = fmaxf(m3, mc);
    if constexpr (TCOPY) {  // staged for the token-contiguous copy
      store16(G2 + lr * kEpiStride2 + c, pg);
      store16(U2 + lr * kEpiStride2 + c, pu);
    }
  };
  // dgu8 is a K-slab [2I/64][ldt][64]; four lanes write one 64-byte row
  const auto store_chunk = [&](int P, int k, const uint32_t (&pg)[4], const uint32_t (&pu)[4]) {
    const int item = 8 * k + wave, slab = item & 3, lr = 16 * (item >> 2) + (lane >> 2);
    const int c = 64 * slab + 16 * (lane & 3);
    const uint32_t o = gu_off(c, half_tile_row(lr, P));
    __builtin_amdgcn_raw_buffer_store_b128(intx4{(int)pg[0], (int)pg[1], (int)pg[2], (int)pg[3]}, rdg, o, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b128(intx4{(int)pu[0], (int)pu[1], (int)pu[2], (int)pu[3]}, rdg,
                                           o + (uint32_t)(I * ldt), 0, 0);
  };
  if constexpr (TCOPY) {
#pragma unroll
    for (int P = 0; P < 2; ++P) {
      gu_loads(P);
      if (P == 1) __syncthreads();  // pass 0's dgu8t copy has read the LDS
      // dh rounded to bf16 (train.py:1082)
      if (P == 0) stage_bf16_half8<0>(DH, acc, 1.0f);
      else stage_bf16_half8<1>(DH, acc, 1.0f);
      __syncthreads();
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        uint32_t pg[4], pu[4];
        swiglu_chunk(P, k, pg, pu);
        store_chunk(P, k, pg, pu);
      }
      __syncthreads();
      // the token-contiguous dgu8t: local rows 0-63 are tile rows 64P.., rows
      // 64-127 tile rows 128 + 64P.. (rows past T hold zero codes)
      const int64_t rp2 = slab_rows(2 * I);
      lds_rows_store_slab_tr<64, 8>(G2, cols, kEpiStride2, dgu8t, rp2, m0 + 64 * P, n0);
      lds_rows_store_slab_tr<64, 8>(G2 + 64 * kEpiStride2, cols, kEpiStride2, dgu8t, rp2, m0 + 128 + 64 * P, n0);
      lds_rows_store_slab_tr<64, 8>(U2, cols, kEpiStride2, dgu8t, rp2, m0 + 64 * P, I + n0);
      lds_rows_store_slab_tr<64, 8>(U2 + 64 * kEpiStride2, cols, kEpiStride2, dgu8t, rp2, m0 + 128 + 64 * P,
                                    I + n0);
    }
    __syncthreads();  // the next tile's DMA overwrites the staging tiles
  } else {
    // Each chunk is stored as soon as its codes are made, so that the stores
    // drain while the rest is computed.  (Deferring the first pass's stores
    // behind the second pass's gu8 requests, so that waiting for those
    // leaves the stores in flight, measured 2 % slower.)  The second pass's
    // gu8 words are requested before its staging.
    uint32_t pg[4][4], pu[4][4];
    gu_loads(0);
    stage_bf16_half8<0>(DH, acc, 1.0f);  // dh rounded to bf16 (train.py:1082)
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      swiglu_chunk(0, k, pg[k], pu[k]);
      store_chunk(0, k, pg[k], pu[k]);
    }
    gu_loads(1);
    __syncthreads();  // every wave has read pass 0's staged rows
    stage_bf16_half8<1>(DH, acc, 1.0f);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      swiglu_chunk(1, k, pg[k], pu[k]);
      store_chunk(1, k, pg[k], pu[k]);
    }
    __syncthreads();  // the next tile's DMA overwrites the staging tile
  }
  }
  m3 *= 1.0f / scale[1];  // s_gu, read again rather than held across the tile loop
  block_amax_atomic<8>(m3, red, amax + 3);
}

// ---------------------------------------------------------------------------
// (a10) gate/up dgrad (spark-gpt train.py:1239-1241):
//   dxn = bf16(acc * (1/s3) * (1/q_gu)), A = d_gu8 (e5m2, [T, 2I]), B = W8^T (e4m3, [D, 2I]).
// One work-group per 256 x 256 tile; the bf16 tile is staged in LDS in two
// passes of 128 rows and written as whole rows.
// With a MoE plan: tile row tm of padded expert order writes its rows(tm)
// valid rows to dxn rows urow(tm).. (expert order, unpadded); W8^T of
// expert e at w8t + e * w_estride, its scale wscale[e].
__global__ __launch_bounds__(512, 1) void gateup_dgrad_kernel(
    const uint8_t* __restrict__ dgu8, const uint8_t* __restrict__ w8t, int64_t T, int64_t D, int64_t I,
    const float* __restrict__ scale, const float* __restrict__ wscale, uint16_t* __restrict__ dxn,
    int64_t ldt, int tiles_m, int tiles_n, const int* __restrict__ plan, int64_t w_estride) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int64_t K = 2 * I;
  const int64_t dp = slab_rows(D);
  int tm, tn;
  // backwards: the dgrad wrote d_gu8 in forward order (0.304 -> 0.302 ms)
  tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn, true);
  int64_t u0 = (int64_t)tm * kTile, uend = T;  // output rows of this tile
  if (plan) {
    const MoePlan P{plan};
    if (tm >= P.ntiles()) return;  // work-group uniform
    const int e = P.expert(tm);
    w8t += e * w_estride;
    wscale += e;
    u0 = P.urow(tm);
    uend = u0 + P.rows(tm);
  }
  const int64_t m0 = (int64_t)tm * kTile, n0 = (int64_t)tn * kTile;
  floatx16 acc[4][2];
  // K-slab operands: dgu8 [2I/64][ldt][64], w8t [2I/64][slab_rows(D)][64]
  MainLoop<false, kFmtE5M2, kFmtE4M3, false, 2, kStages, 0, false, false, 4>::run(
      lds, dgu8 + m0 * kStage, K * ldt - m0 * kStage, [=](int r) { return r * kStage; }, (int)(ldt * kStage),
      w8t + n0 * kStage, K * dp - n0 * kStage, [=](int r) { return plain_col_nb<2>(r) * kStage; },
      (int)(dp * kStage), (int)(K / kStage), acc);
  // the scales are read after the K loop, so that nothing is held across it
  const float sab = (1.0f / scale[3]) * (1.0f / wscale[0]);  // both powers of two
  stage_bf16_half8<0>(lds, acc, sab);
  __syncthreads();
  write_bf16_half<512>(lds, 0, u0, n0, uend, D, D, dxn);
  __syncthreads();
  stage_bf16_half8<1>(lds, acc, sab);
  __syncthreads();
  write_bf16_half<512>(lds, 1, u0, n0, uend, D, D, dxn);
}

// ---------------------------------------------------------------------------
// (a12, a13) weight gradients, reduced over tokens:
//   out[m, n] = sum_t A[m, t] * B[n, t] / (sa * sb)
// A, B are K-slab token-contiguous fp8 copies (common.h) over ldt tokens
// (zeros past T): a tile's K stage is one contiguous 16 KiB block of each.
// The grid is tiles * splits work-groups (split_tile_coords); split sp takes
// K bytes [sp * kchunk, min((sp + 1) * kchunk, ldt)) (the last split may be
// shorter; every split is a whole number of 128-byte stage pairs); with splits > 1
// each split writes its raw fp32 accumulators to ws in accumulator order
// (frag_offset below: each wave store instruction is one contiguous 1 KiB
// run) and splitk_reduce_kernel sums them in split order (deterministic) and
// scatters them to [M, N].
// With `partials` (and always with BF16) the raw partials go to `out` as the
// workspace, also for one split (the reductions that round to bf16 or apply
// the optimizer's momentum stage).  BF16: bf16 operands (2 bytes per token:
// `ldt` and `kchunk` count K bytes).
// TRA / TRB: that operand is instead a row K-slab of the token-major
// activation ([M/64][ldt][64] or [N/64][ldt][64]: h8 and dgu8 as their
// producers write them for the forward GEMMs), read through transposing LDS
// reads (MainLoop TR_A / TR_B); the partials then always go to `out` as the
// workspace, in the same order (with TRB the columns unpermuted:
// splitk_reduce_kernel<true>).
// NW = 4 waves (one per SIMD) of 128 x 128, or 8 (two per SIMD) of 128 x 64,
// so that one wave's stage waits and barriers are covered by the other's
// MFMAs; the accumulator order follows the wave shape (acc_order_rc).
// Addressing of a transposed-read operand: row r of block r / 64 (fp8) or
// r / 32 (bf16) at token t lies at base + block * bs + t * ts, and ext bytes
// are readable from base (the rest reads as zero).  A row K-slab of [T, L]
// over ldt tokens: ts = 64, bs = ldt * 64; row-major [T, L] rows: ts = the row
// bytes, bs = 64, ext = T * ts.
struct TrOp {
  int64_t ts, bs, ext;
};

// Waves per work-group of the weight gradients (FP8 and bf16).
constexpr int kWgradWaves = 8;
constexpr int kBf16WgradWaves = 8;

template <bool BF16, int FMT_A, int FMT_B, bool TRA = false, bool TRB = false, int NW = 4>
__global__ __launch_bounds__(64 * NW, 1) void wgrad_kernel(
    const uint8_t* __restrict__ at, const uint8_t* __restrict__ bt, int64_t M, int64_t N, int64_t ldt,
    int64_t kchunk, const float* __restrict__ sa, const float* __restrict__ sb, float* __restrict__ out,
    int tiles_m, int tiles_n, int splits, int partials, TrOp tra, TrOp trb) {
  static_assert(NW == 4 || NW == 8, "4 or 8 waves");
  constexpr int NB = NW == 8 ? 2 : 4, WN = NW / 2;  // B blocks of 32 per wave, wave columns
  extern __shared__ __align__(16) uint8_t lds[];
  int tm, tn, sp;
  split_tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, splits, tm, tn, sp);
  if (sp >= splits) return;  // grid padding (work-group uniform)
  const int64_t m0 = (int64_t)tm * kTile, n0 = (int64_t)tn * kTile;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  floatx16 acc[4][NB];
  const int64_t kb = (int64_t)sp * kchunk;
  {
    // K-slab operands: slab (kb / 64) of A starts at (kb / 64) * rpa * 64.
    // TR operands (TrOp): tile row r is row r % kRows of block r / kRows at
    // the stage's tokens; a stage (64 K bytes: kRows tokens) is kRows * ts on.
    constexpr int kRows = BF16 ? 32 : 64;
    const int64_t rpa = slab_rows(M), rpb = slab_rows(N);
    const int64_t t0 = kb / (BF16 ? 2 : 1);  // first token of the split
    const int ats = (int)tra.ts, abs_ = (int)tra.bs, bts = (int)trb.ts, bbs = (int)trb.bs;
    const uint8_t* a0 = TRA ? at + (m0 / kRows) * tra.bs + t0 * tra.ts : at + (kb / kStage) * rpa * kStage + m0 * kStage;
    const uint8_t* b0 = TRB ? bt + (n0 / kRows) * trb.bs + t0 * trb.ts : bt + (kb / kStage) * rpb * kStage + n0 * kStage;
    const uint8_t* a_end = TRA ? at + tra.ext : at + ldt * rpa;
    const uint8_t* b_end = TRB ? bt + trb.ext : bt + ldt * rpb;
    MainLoop<BF16, FMT_A, FMT_B, false, NB, kStages, 0, TRA, TRB, WN>::run(
        lds, a0, a_end - a0, [=](int r) { return TRA ? (r / kRows) * abs_ + (r % kRows) * ats : r * kStage; },
        TRA ? kRows * ats : (int)(rpa * kStage), b0, b_end - b0,
        [=](int r) { return TRB ? (r / kRows) * bbs + (r % kRows) * bts : plain_col_nb<NB>(r) * kStage; },
        TRB ? kRows * bts : (int)(rpb * kStage), (int)((kchunk < ldt - kb ? kchunk : ldt - kb) / kStage), acc);
  }
  if (BF16 || TRA || TRB || partials) {
    // accumulator order: [split][tile][wave][tb][nb][i][lane][4]
    float* frag = out + ((int64_t)sp * tiles_m * tiles_n + (int64_t)tm * tiles_n + tn) * (kTile * kTile) +
                  wave * (kTile * kTile / NW);
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          reinterpret_cast<floatx4*>(frag + (tb * NB + nb) * 1024 + i * 256)[lane] =
              floatx4{acc[tb][nb][4 * i], acc[tb][nb][4 * i + 1], acc[tb][nb][4 * i + 2], acc[tb][nb][4 * i + 3]};
    return;
  }
  const float deq = 1.0f / (sa[0] * sb[0]);
  float* dst = out;
  const int fr = lane & 31, g = lane >> 5;
  const int cb = 32 * NB * wn + 16 * NB * g;  // plain_col_nb<NB>
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    const int64_t m = m0 + 128 * wm + 32 * tb + fr;
    if (m >= M) continue;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int64_t n = n0 + cb + 16 * nb;
      floatx4* p = reinterpret_cast<floatx4*>(dst + m * N + n);
      // N % 4 == 0: each float4 is wholly inside the row or wholly past it
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (n + 4 * i < N)
          p[i] = floatx4{acc[tb][nb][4 * i] * deq, acc[tb][nb][4 * i + 1] * deq, acc[tb][nb][4 * i + 2] * deq,
                         acc[tb][nb][4 * i + 3] * deq};
    }
  }
}

// Grouped (MoE) weight gradient: out[e, m, n] = sum over expert e's padded
// rows t of A[m, t] * B[n, t] / (sa * sb), A and B token-contiguous K-slab
// copies over the padded expert order (zeros in padding rows).  Work-group
// Work-group (expert e, split sp, tile) of a 1-D grid over the three, tile
// fastest, takes split sp of the expert's 64-token stages (an even number of
// them; none for an expert without rows, whose gradient comes out zero).
// Each XCD takes a contiguous run of that order, so the work-groups resident
// on one XCD share one (expert, split) K range of A and B in its L2 (with the
// tile index spread over the XCDs, every XCD read every expert's operands:
// 3.9x the algorithmic bytes at the MoE workload).  With one split it
// writes out[e] itself; otherwise its raw partial in accumulator order to
// ws[e][sp][tile], summed in split order by splitk_reduce_kernel.
// BF16: bf16 operands, 2 bytes per padded row (`ldp` counts K bytes), and the
// partials always go to ws, for bf16_wgrad_reduce_kernel to round.
template <bool BF16, int FMT_A, int FMT_B, bool TRA = false, bool TRB = false, int NW = 4>
__global__ __launch_bounds__(64 * NW, 1) void moe_wgrad_kernel(
    const uint8_t* __restrict__ at, const uint8_t* __restrict__ bt, int64_t M, int64_t N, int64_t ldp,
    const float* __restrict__ sa, const float* __restrict__ sb, float* __restrict__ out, float* __restrict__ ws,
    const int* __restrict__ plan, int tiles_m, int tiles_n, int splits) {
  static_assert(NW == 4 || NW == 8, "4 or 8 waves (as wgrad_kernel)");
  constexpr int NB = NW == 8 ? 2 : 4, WN = NW / 2;
  extern __shared__ __align__(16) uint8_t lds[];
  const MoePlan P{plan};
  const int tiles = tiles_m * tiles_n;
  const int lid = xcd_run(blockIdx.x, gridDim.x);
  const int sp = (lid / tiles) % splits, e = lid / (tiles * splits);
  int tm, tn;
  raster(lid % tiles, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * kTile, n0 = (int64_t)tn * kTile;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  constexpr int64_t kBpe = BF16 ? 2 : 1;  // K bytes per padded row
  const int64_t nst = P.pcount(e) * kBpe / kStage;  // a multiple of 4
  int64_t q = (nst + splits - 1) / splits;
  q = (q + 1) & ~(int64_t)1;
  const int64_t k0 = (int64_t)sp * q;
  const int64_t nk = nst - k0 < 0 ? 0 : (nst - k0 < q ? nst - k0 : q);
  const int64_t rpa = slab_rows(M), rpb = slab_rows(N);
  const int64_t s0 = P.pstart(e) * kBpe / kStage + k0;  // first 64-byte stage
  // Token-contiguous operands: stage s at s * rows * 64.  Row K-slab (TR)
  // operands ([rows/kRows][padded rows][64], as for wgrad_kernel): tile row r
  // is token r % kRows of slab r / kRows, and a stage (kRows tokens) is
  // kRows * 64 bytes on in every slab.
  constexpr int kRows = BF16 ? 32 : 64;
  const int64_t ldt_tok = ldp / kBpe;  // padded rows (ldp counts K bytes)
  const int ltok = (int)ldt_tok;
  const uint8_t* a0 = TRA ? at + (m0 / kRows) * ldt_tok * kStage + s0 * kRows * kStage : at + s0 * rpa * kStage + m0 * kStage;
  const uint8_t* b0 = TRB ? bt + (n0 / kRows) * ldt_tok * kStage + s0 * kRows * kStage : bt + s0 * rpb * kStage + n0 * kStage;
  const uint8_t* a_end = TRA ? at + (M / kRows) * ldt_tok * kStage : at + ldp * rpa;
  const uint8_t* b_end = TRB ? bt + (N / kRows) * ldt_tok * kStage : bt + ldp * rpb;
  const int64_t a_bytes = nk > 0 ? a_end - a0 : 0, b_bytes = nk > 0 ? b_end - b0 : 0;
  floatx16 acc[4][NB];
  MainLoop<BF16, FMT_A, FMT_B, false, NB, kStages, 0, TRA, TRB, WN>::run(
      lds, a0, a_bytes, [=](int r) { return TRA ? ((r / kRows) * ltok + (r % kRows)) * kStage : r * kStage; },
      TRA ? kRows * kStage : (int)(rpa * kStage), b0, b_bytes,
      [=](int r) { return TRB ? ((r / kRows) * ltok + (r % kRows)) * kStage : plain_col_nb<NB>(r) * kStage; },
      TRB ? kRows * kStage : (int)(rpb * kStage), (int)nk, acc);
  if (BF16 || TRA || TRB || splits > 1) {
    // accumulator order: [expert][split][tile][wave][tb][nb][i][lane][4]
    float* frag = ws + (((int64_t)e * splits + sp) * tiles_m * tiles_n + (int64_t)tm * tiles_n + tn) * (kTile * kTile) +
                  wave * (kTile * kTile / NW);
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          reinterpret_cast<floatx4*>(frag + (tb * NB + nb) * 1024 + i * 256)[lane] =
              floatx4{acc[tb][nb][4 * i], acc[tb][nb][4 * i + 1], acc[tb][nb][4 * i + 2], acc[tb][nb][4 * i + 3]};
    return;
  }
  const float deq = 1.0f / (sa[0] * sb[0]);
  float* dst = out + (int64_t)e * M * N;
  const int fr = lane & 31, g = lane >> 5;
  const int cb = 32 * NB * wn + 16 * NB * g;  // plain_col_nb<NB>
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    const int64_t m = m0 + 128 * wm + 32 * tb + fr;
    if (m >= M) continue;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int64_t n = n0 + cb + 16 * nb;
      floatx4* p = reinterpret_cast<floatx4*>(dst + m * N + n);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (n + 4 * i < N)
          p[i] = floatx4{acc[tb][nb][4 * i] * deq, acc[tb][nb][4 * i + 1] * deq, acc[tb][nb][4 * i + 2] * deq,
                         acc[tb][nb][4 * i + 3] * deq};
    }
  }
}

// out[0, n) = 0: four floats per thread (n % 4 == 0, out 16-byte aligned).
__global__ __launch_bounds__(256) void zero_fill_kernel(float* __restrict__ out, int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i < n) *reinterpret_cast<floatx4*>(out + i) = floatx4{0.f, 0.f, 0.f, 0.f};
}

// Tile row r and column c of the first value of float4 q (< 16384) of one
// 256 x 256 partial tile of wgrad_kernel<.., NW> in accumulator order
// [wave][tb][nb][i][lane][4] (NB = 4 or 2 blocks of 32 columns per wave;
// wave (wm, wn) = (wave & 1, wave >> 1) owns rows 128 wm.. and columns
// 32 NB wn..): B-tile rows permuted by plain_col_nb<NB> (accumulator v of
// block nb, lane half g is column 32 NB wn + 16 NB g + 16 nb + v), or with
// TR_B unpermuted (column 32 NB wn + 32 nb + 8 (v / 4) + 4 g + v % 4).
template <int NW, bool TR_B>
SFP8_DEV void acc_order_rc(int q, int& r, int& c) {
  constexpr int NB = NW == 8 ? 2 : 4, NBB = NW == 8 ? 1 : 2;
  const int lane = q & 63, i = (q >> 6) & 3, nb = (q >> 8) & (NB - 1), tb = (q >> (8 + NBB)) & 3;
  const int wave = (q >> (10 + NBB)) & (NW - 1), g = lane >> 5;
  r = 128 * (wave & 1) + 32 * tb + (lane & 31);
  c = 32 * NB * (wave >> 1) + (TR_B ? 32 * nb + 8 * i + 4 * g : 16 * NB * g + 16 * nb + 4 * i);
}

// Split-K reduction of the accumulator-order partials of wgrad_kernel:
// out[m, n] = (sum over s ascending of ws[s]) / (sa * sb).  Thread q owns the
// q-th float4 of one split's partials; its (m, n) follows from the MFMA
// accumulator layout (acc_order_rc; TR_B: partials of wgrad_kernel<..,
// true>).
template <bool TR_B = false, int NW = 4>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ ws, int splits,
                                                            int64_t n4, int tiles_n, int64_t M, int64_t N,
                                                            const float* __restrict__ sa,
                                                            const float* __restrict__ sb, float* __restrict__ out) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (q >= n4) return;
  // expert blockIdx.y of a grouped gradient: its splits' partials, its [M, N]
  ws += (int64_t)blockIdx.y * splits * n4 * 4;
  out += (int64_t)blockIdx.y * M * N;
  const floatx4* w4 = reinterpret_cast<const floatx4*>(ws);
  floatx4 acc = __builtin_nontemporal_load(w4 + q);
  for (int s = 1; s < splits; ++s) acc += __builtin_nontemporal_load(w4 + (int64_t)s * n4 + q);
  int r, c;
  acc_order_rc<NW, TR_B>((int)(q & 16383), r, c);
  const int64_t tile = q >> 14;
  const int64_t tm = tile / tiles_n, tn = tile % tiles_n;
  const int64_t m = tm * kTile + r, n = tn * kTile + c;
  if (m < M && n < N) {
    const float deq = 1.0f / (sa[0] * sb[0]);
    *reinterpret_cast<floatx4*>(out + m * N + n) = acc * deq;
  }
}

// ---------------------------------------------------------------------------
// bf16 SwiGLU MLP path (spark-gpt's default, non-FP8 path): the gate/up GEMM
// with the SwiGLU epilogue of _swiglu_gemm_kernel (train.py:1625-1716), the
// plain bf16 GEMM of its dgrad and the rounding reduce of its weight
// gradient.  Operands are bf16 K-slabs (2 bytes per element: a 64-byte
// stage is 32 elements of K) or, for the forward's A, the caller's
// row-major x.

// Forward: gate/up = x @ W^T per tile (fp32 accumulate), then
//   g = bf16(acc_g * rs), u = bf16(acc_u * rs)   (rs = rstd[row] when the
//   RMSNorm is folded into W, else 1; train.py:1696-1702),
//   h = bf16(g * sigmoid(g) * u)                (train.py:1709-1715),
// gu = [g | u] row-major [rows, 2I] (saved for the backward), h row-major
// [rows, I].  Tile: 256 rows x 128 (gate, up) column pairs; B is the bf16
// K-slab of W [2D/64][slab_rows(2I)][64] in the paired layout (a lane holds
// g and u of the same 32 consecutive columns).  A = x row-major [rows, D]
// (rows past the tile's last read as zero through the range check).
// With a MoE plan: tile row tm of padded expert order reads and writes the
// expert-order rows urow(tm) .. + rows(tm); W of expert e at w + e * w_estride
// (bytes).  Columns from I on (the last tile when I % 128 != 0) are not
// written.
constexpr int kGuStride = 272;  // staging row: 128 bf16 columns (256 bytes) + 16

// 8 waves (two per SIMD): wave (wm, wn) owns tile rows 128*wm.. and one
// 32-column block of gate and one of up, columns 32*wn.. of each half.
__global__ __launch_bounds__(512, 1) void bf16_swiglu_fwd_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ w, int64_t T, int64_t D, int64_t I,
    const float* __restrict__ rstd, uint16_t* __restrict__ gu, uint16_t* __restrict__ h, int tiles_m, int tiles_n,
    const int* __restrict__ plan, int64_t w_estride, int64_t ldxs) {
  extern __shared__ __align__(16) uint8_t lds[];
  int tm, tn;
  tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
  int64_t r0 = (int64_t)tm * kTile, nrows = T - r0;
  if (plan) {
    const MoePlan P{plan};
    if (tm >= P.ntiles()) return;  // work-group uniform
    r0 = P.urow(tm);
    nrows = P.rows(tm);
    w += P.expert(tm) * w_estride;
  }
  const int64_t n0 = (int64_t)tn * 128;
  const int64_t ldx = D * 2;  // bytes per x row = K bytes
  const int64_t wr = slab_rows(2 * I);
  // the outputs from the tile's first row (gu [rows, 2I], h [rows, I], bf16)
  const __amdgpu_buffer_rsrc_t rgu = make_rsrc(gu + r0 * 2 * I, nrows * 4 * I);
  const __amdgpu_buffer_rsrc_t rho = make_rsrc(h + r0 * I, nrows * 2 * I);
  floatx16 acc[4][2];  // [tb][0] gate, [tb][1] up
  // A: x row-major [T, D] (rows past the tile's last read as zero through
  // the range check), or with ldxs > 0 its row K-slab [2D/64][ldxs][64]
  // (zero padding rows): a K stage of the tile is then one 16 KiB block of
  // whole 128-byte lines instead of 256 half lines 2D bytes apart
  const bool xslab = ldxs > 0;
  MainLoop<true, 0, 0, true, 2, kStages, 0, false, false, 4>::run(
      lds, reinterpret_cast<const uint8_t*>(x) + r0 * (xslab ? kStage : ldx),
      xslab ? ldx * ldxs - r0 * kStage : nrows * ldx, [=](int r) { return r * (xslab ? kStage : (int)ldx); },
      xslab ? (int)(ldxs * kStage) : kStage, w, ldx * wr, [=](int r) { return ((r >> 7) * (int)I + (int)n0 + paired_col8(r)) * kStage; },
      (int)(wr * kStage), (int)(ldx / kStage), acc);
  // Epilogue in two passes of 128 tile rows: pass P takes the lanes' row
  // blocks tb = 2P, 2P+1 (tile row 128 wm + 64 P + 32 (tb & 1) + fr, staging
  // row 64 wm + 32 (tb & 1) + fr), stages g, u and h as bf16 rows in LDS,
  // then writes them as whole 256-byte row runs.
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave & 1, wn = wave >> 1, fr = lane & 31, g = lane >> 5;
  const int cb = 32 * wn + 16 * g;  // first of this lane's 16 columns in the tile
  uint8_t* Gs = lds;
  uint8_t* Us = lds + 128 * kGuStride;
  uint8_t* Hs = lds + 2 * 128 * kGuStride;
  const float c_exp = -1.4426950408889634f;
#pragma unroll
  for (int P = 0; P < 2; ++P) {
    if (P) __syncthreads();  // the first pass's rows are out of the staging tiles
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int tb = 2 * P + q;
      const int lr = 128 * wm + 32 * tb + fr;  // row within the tile
      const float rs = (rstd && lr < nrows) ? rstd[r0 + lr] : 1.0f;
      uint32_t gw[8], uw[8], hw[8];
#pragma unroll
      for (int v = 0; v < 16; v += 2) {
        const uint32_t pg = pack2_bf16(acc[tb][0][v] * rs, acc[tb][0][v + 1] * rs);
        const uint32_t pu = pack2_bf16(acc[tb][1][v] * rs, acc[tb][1][v + 1] * rs);
        const float g0 = __uint_as_float(pg << 16), g1 = __uint_as_float(pg & 0xffff0000u);
        const float u0 = __uint_as_float(pu << 16), u1 = __uint_as_float(pu & 0xffff0000u);
        const float s0 = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g0 * c_exp));
        const float s1 = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g1 * c_exp));
        const int k = v / 2;
        gw[k] = pg;
        uw[k] = pu;
        hw[k] = pack2_bf16(g0 * s0 * u0, g1 * s1 * u1);
      }
      const int sr = 64 * wm + 32 * q + fr;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        store16(Gs + sr * kGuStride + 2 * cb + 16 * j, {gw[4 * j], gw[4 * j + 1], gw[4 * j + 2], gw[4 * j + 3]});
        store16(Us + sr * kGuStride + 2 * cb + 16 * j, {uw[4 * j], uw[4 * j + 1], uw[4 * j + 2], uw[4 * j + 3]});
        store16(Hs + sr * kGuStride + 2 * cb + 16 * j, {hw[4 * j], hw[4 * j + 1], hw[4 * j + 2], hw[4 * j + 3]});
      }
    }
    __syncthreads();
    // 128 rows x 16 pieces of 16 bytes per output: sixteen lanes per row;
    // buffer stores from the tile's first row, a piece past the valid rows or
    // past I (I % 8 == 0: whole pieces) at offset 2^31 (beyond the range:
    // dropped), so every thread issues the same stores without a branch
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int idx = (int)threadIdx.x + 512 * k;
      const int sr = idx >> 4, c = idx & 15;
      const int lr = half_tile_row(sr, P);
      const int64_t col = n0 + 8 * c;
      const uint32_t in = 0u - (uint32_t)(lr < nrows && col < I);
      const uint32_t og = ((uint32_t)((lr * 2 * I + col) * 2) & in) | (~in & 0x80000000u);
      const uint32_t oh = ((uint32_t)((lr * I + col) * 2) & in) | (~in & 0x80000000u);
      __builtin_amdgcn_raw_buffer_store_b128(*reinterpret_cast<const intx4*>(Gs + sr * kGuStride + 16 * c), rgu,
                                             og, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b128(*reinterpret_cast<const intx4*>(Us + sr * kGuStride + 16 * c), rgu,
                                             og + (uint32_t)(2 * I), 0, 0);
      __builtin_amdgcn_raw_buffer_store_b128(*reinterpret_cast<const intx4*>(Hs + sr * kGuStride + 16 * c), rho,
                                             oh, 0, 0);
    }
  }
}

// out[u, n] = bf16(sum_k A[m, k] * B[n, k]) with A a bf16 K-slab over lda
// rows (Kb bytes of K) and B a bf16 K-slab [Kb/64][slab_rows(N)][64]: the
// dgrad of the SwiGLU path (_swiglu_dgrad_kernel, train.py:1907-1980, its
// d_gu operand precomputed).  One work-group per 256 x 256 tile; the bf16
// tile is staged in LDS in two passes of 128 rows and written as whole rows.
// With a MoE plan: A in padded expert order, tile row tm writes its rows(tm)
// valid rows to out rows urow(tm).. (expert order); B of expert e at
// b + e * b_estride (bytes).
// 8 waves (two per SIMD), each 128 x 64.
__global__ __launch_bounds__(512, 1) void bf16_gemm_kernel(
    const uint8_t* __restrict__ a, const uint8_t* __restrict__ b, int64_t T, int64_t N, int64_t Kb, int64_t lda,
    uint16_t* __restrict__ out, int tiles_m, int tiles_n, const int* __restrict__ plan, int64_t b_estride) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int64_t bp = slab_rows(N);
  int tm, tn;
  tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
  int64_t u0 = (int64_t)tm * kTile, uend = T;  // output rows of this tile
  if (plan) {
    const MoePlan P{plan};
    if (tm >= P.ntiles()) return;  // work-group uniform
    b += P.expert(tm) * b_estride;
    u0 = P.urow(tm);
    uend = u0 + P.rows(tm);
  }
  const int64_t m0 = (int64_t)tm * kTile, n0 = (int64_t)tn * kTile;
  floatx16 acc[4][2];
  MainLoop<true, 0, 0, false, 2, kStages, 0, false, false, 4>::run(
      lds, a + m0 * kStage, Kb * lda - m0 * kStage, [=](int r) { return r * kStage; }, (int)(lda * kStage),
      b + n0 * kStage, Kb * bp - n0 * kStage, [=](int r) { return plain_col_nb<2>(r) * kStage; }, (int)(bp * kStage),
      (int)(Kb / kStage), acc);
  stage_bf16_half8<0>(lds, acc, 1.0f);
  __syncthreads();
  write_bf16_half<512>(lds, 0, u0, n0, uend, N, N, out);
  __syncthreads();
  stage_bf16_half8<1>(lds, acc, 1.0f);
  __syncthreads();
  write_bf16_half<512>(lds, 1, u0, n0, uend, N, N, out);
}

// The bf16 weight gradient's reduction: out[m, n] = bf16(sum over s
// ascending of ws[s]) (the bf16 result of _swiglu_wgrad_kernel,
// train.py:1983-2026), partials in wgrad_kernel's accumulator order;
// blockIdx.y = expert of a grouped gradient (out [E, M, N]).
template <bool TR_B = false, int NW = 4>
__global__ __launch_bounds__(256) void bf16_wgrad_reduce_kernel(const float* __restrict__ ws, int splits, int64_t n4,
                                                                int tiles_n, int64_t M, int64_t N,
                                                                uint16_t* __restrict__ out) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (q >= n4) return;
  ws += (int64_t)blockIdx.y * splits * n4 * 4;
  out += (int64_t)blockIdx.y * M * N;
  const floatx4* w4 = reinterpret_cast<const floatx4*>(ws);
  floatx4 acc = __builtin_nontemporal_load(w4 + q);
  for (int s = 1; s < splits; ++s) acc += __builtin_nontemporal_load(w4 + (int64_t)s * n4 + q);
  int r, c;
  acc_order_rc<NW, TR_B>((int)(q & 16383), r, c);
  const int64_t tile = q >> 14;
  const int64_t tm = tile / tiles_n, tn = tile % tiles_n;
  const int64_t m = tm * kTile + r, n = tn * kTile + c;
  if (m < M && n < N)  // N % 4 == 0: the 4 values are wholly inside or past the row
    *reinterpret_cast<intx2*>(out + m * N + n) = intx2{(int)pack2_bf16(acc[0], acc[1]), (int)pack2_bf16(acc[2], acc[3])};
}

// The weight gradient with the optimizer's momentum stage fused into its
// reduction (the consumer of dW, train.py:2805-2820, applied as the split
// sum leaves the registers): d = (sum over s ascending of ws[s]) / (sa * sb),
// then v <- lerp(v, d, w_v) in place and u = bf16(lerp(d, v, 1 - w_u1)) into
// the Newton-Schulz staging matrix ([M, N] bf16, the parameter's layout);
// grad[m, n] = d when grad is given.  splits == 0: d = 0 (no tokens).  TR_B:
// the partials' columns are in the transposed-read B order, as for
// splitk_reduce_kernel<true>; NW: the partials of wgrad_kernel<.., NW>.
template <bool TR_B = false, int NW = 4>
__global__ __launch_bounds__(256) void splitk_momentum_kernel(const float* __restrict__ ws, int splits, int64_t n4,
                                                              int tiles_n, int64_t M, int64_t N,
                                                              const float* __restrict__ sa,
                                                              const float* __restrict__ sb, float* __restrict__ grad,
                                                              float* __restrict__ v, uint16_t* __restrict__ u,
                                                              float w_v, float w_u1) {
  // Work-group b sums the b-th 256 float4s of every split: a 32 x 32 block of
  // dW (fixed tile, wave, row block tb, column block nb), passed through LDS
  // so that eight lanes then cover 32 contiguous columns of one row of v, u
  // and grad (n4 is a multiple of 256: no partial work-group).
  __shared__ floatx4 blk[32][9];
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const floatx4* w4 = reinterpret_cast<const floatx4*>(ws);
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < splits; ++s) acc += __builtin_nontemporal_load(w4 + (int64_t)s * n4 + q);
  constexpr int NB = NW == 8 ? 2 : 4, NBB = NW == 8 ? 1 : 2;
  const int lane = threadIdx.x & 63, i = threadIdx.x >> 6;
  const int64_t b = blockIdx.x;
  const int nb = (int)(b & (NB - 1)), tb = (int)(b >> NBB) & 3, wave = (int)(b >> (NBB + 2)) & (NW - 1);
  const int64_t tile = b >> 6;
  const int64_t tm = tile / tiles_n, tn = tile % tiles_n;
  // local column (0..31) of this thread's float4 in the block
  const int c = TR_B ? 8 * i + 4 * (lane >> 5) : 16 * (lane >> 5) + 4 * i;
  blk[lane & 31][c >> 2] = acc * (1.0f / (sa[0] * sb[0]));
  __syncthreads();
  const int r = threadIdx.x >> 3, c2 = 4 * (threadIdx.x & 7);
  const int64_t m = tm * kTile + 128 * (wave & 1) + 32 * tb + r;
  // local column -> output column: TR_B blocks are 32 contiguous columns,
  // the plain layout's two 16-column halves lie 16 NB columns apart
  const int64_t n =
      tn * kTile + 32 * NB * (wave >> 1) + (TR_B ? 32 * nb + c2 : 16 * nb + (c2 < 16 ? c2 : 16 * NB - 16 + c2));
  if (m >= M || n >= N) return;
  const floatx4 d = blk[r][c2 >> 2];
  if (grad) *reinterpret_cast<floatx4*>(grad + m * N + n) = d;
  floatx4 vv = *reinterpret_cast<const floatx4*>(v + m * N + n);
  uint32_t uu[2];
  momentum4(d, vv, w_v, w_u1, uu);
  *reinterpret_cast<floatx4*>(v + m * N + n) = vv;
  *reinterpret_cast<intx2*>(u + m * N + n) = intx2{(int)uu[0], (int)uu[1]};
}

}  // namespace sfp8

static_assert(3 * sfp8::kTile * sfp8::kEpiStride + 64 <= sfp8::kMainLds, "swiglu epilogue tiles fit the main loop's LDS");
static_assert(sfp8::kPipeLds <= 160 * 1024, "deferred-epilogue SwiGLU fits the 160 KiB LDS");
static_assert(128 * sfp8::kBf16Stride <= sfp8::kMainLds, "bf16 epilogue staging fits the main loop's LDS");
static_assert(3 * 128 * sfp8::kGuStride <= sfp8::kMainLds, "bf16 SwiGLU staging fits the main loop's LDS");

// ============================================================================
// C ABI
// ============================================================================
using namespace sfp8;

namespace {

// epilogue tiles (2 x 256 x 272) + 4 amax floats, or the main loop's ring
constexpr int kDgradEpiLds = 2 * kTile * kEpiStride2 + 32;
constexpr int kDgradLds = kDgradLutBytes + (kDgradEpiLds > kMainLds ? kDgradEpiLds : kMainLds);

template <typename K>
int prep(K kernel, int lds_bytes) {
  // dynamic LDS above 64 KiB must be opted into once per kernel
  const hipError_t e = hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           lds_bytes);
  return e == hipSuccess ? kOk : (int)e;
}

inline int status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? kOk : (int)e;
}

inline bool al16(const void* p) { return (((uintptr_t)p) & 15u) == 0; }
inline int cdiv(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

// Compute units of the current device (queried on every call: no cached state).
inline int cu_count(int* n) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(n, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return (int)e;
  if (*n <= 0) *n = 1;
  return 0;
}
// offsets inside one operand tile are 32-bit
inline bool fits32(int64_t rows, int64_t ld) { return rows * ld < (int64_t)1 << 31; }

// Work-groups launched for a split-K weight gradient of `tiles` tiles: when
// padding the grid to whole 32-tile runs per XCD (256 work-groups a round)
// adds no round of work-groups, it is padded, so that every round of an XCD
// runs 32 consecutive tiles of one split (one raster group of 8 tile rows x
// 4 tile columns at 4 tile columns); the padding work-groups exit at once.
inline int wgrad_grid(int tiles, int splits) {
  const int n = tiles * splits, padded = (n + 255) / 256 * 256;
  return splits > 1 && (tiles % 32) == 0 ? padded : n;
}

// K bytes per weight-gradient split: ldt / s rounded up to whole 128-byte
// stage pairs (the last split takes what remains).
inline int64_t wgrad_chunk(int64_t ldt, int64_t s) {
  const int64_t per = (ldt + s - 1) / s;
  return (per + 2 * kStage - 1) / (2 * kStage) * (2 * kStage);
}

}  // namespace

namespace {
// The split partials ws[split][tile] (one 256 x 256 fp32 tile each, in
// accumulator order of wgrad_kernel<.., kWgradWaves>) of the FP8 weight
// gradient; TRA / TRB: that operand is the row K-slab of the token-major
// activation instead of a token-contiguous copy.
template <bool TRA, bool TRB>
int wgrad_partials(const void* a, const void* b, int64_t M, int64_t N, int64_t ldt, const float* sa, const float* sb,
                   float* ws, int splits, hipStream_t st) {
  const int tiles_m = cdiv(M, kTile), tiles_n = cdiv(N, kTile);
  const int rc = prep(wgrad_kernel<false, kFmtE5M2, kFmtE4M3, TRA, TRB, kWgradWaves>, kMainLds);
  if (rc) return rc;
  // row K-slabs over ldt tokens
  const TrOp tra{kStage, ldt * kStage, (M / 64) * ldt * kStage}, trb{kStage, ldt * kStage, (N / 64) * ldt * kStage};
  hipLaunchKernelGGL((wgrad_kernel<false, kFmtE5M2, kFmtE4M3, TRA, TRB, kWgradWaves>),
                     dim3((unsigned)wgrad_grid(tiles_m * tiles_n, splits)), dim3(64 * kWgradWaves), kMainLds, st, (const uint8_t*)a, (const uint8_t*)b, M, N, ldt, wgrad_chunk(ldt, splits), sa,
                     sb, ws, tiles_m, tiles_n, splits, 1, tra, trb);
  return status();
}

int wgrad_partials_any(bool a_rows, bool b_rows, const void* a, const void* b, int64_t M, int64_t N, int64_t ldt,
                       const float* sa, const float* sb, float* ws, int splits, hipStream_t st) {
  if (a_rows && b_rows) return wgrad_partials<true, true>(a, b, M, N, ldt, sa, sb, ws, splits, st);
  if (a_rows) return wgrad_partials<true, false>(a, b, M, N, ldt, sa, sb, ws, splits, st);
  if (b_rows) return wgrad_partials<false, true>(a, b, M, N, ldt, sa, sb, ws, splits, st);
  return wgrad_partials<false, false>(a, b, M, N, ldt, sa, sb, ws, splits, st);
}
}  // namespace

extern "C" {

int sfp8_gemm_gateup_swiglu_fwd(const void* x8, const void* w8, int64_t T, int64_t D, int64_t I,
                                const float* scale, const float* wscale, float* amax, void* gu8, void* h8,
                                void* h8t, int64_t ldt, void* stream) {
  // token-sized buffers may be null when there are no tokens
  if (!w8 || !scale || !wscale || !amax || (T > 0 && (!x8 || !gu8 || !h8))) return kErrNullPointer;
  // the grid covers ceil(T / 256) token tiles, which write every padding
  // token of the outputs only when ldt is T rounded up to 256
  if (T < 0 || D <= 0 || I <= 0 || D % (2 * kStage) || I % 128 || ldt != (int64_t)cdiv(T, kTile) * kTile)
    return kErrBadShape;
  if (!fits32(ldt, D) || !fits32(2 * I, D) || !fits32(ldt, I) || !fits32(ldt, 2 * I)) return kErrBadShape;
  if (!al16(x8) || !al16(w8) || !al16(gu8) || !al16(h8) || !al16(h8t)) return kErrBadAlignment;
  if (T == 0) return kOk;
  if (D == 1024) {
    // persistent, one work-group per CU, SwiGLU of each tile overlapped with
    // the next tile's K loop
    const int tiles_m = cdiv(T, kTile), tiles_n = (int)(I / 64);
    const int ntiles = tiles_m * tiles_n;
    int n_cu = 0;
    int rc = cu_count(&n_cu);
    if (rc) return rc;
    rc = prep(swiglu_pipe_kernel<16, kPipeTB>, kPipeLds);
    if (rc) return rc;
    hipLaunchKernelGGL((swiglu_pipe_kernel<16, kPipeTB>), dim3(ntiles < n_cu ? ntiles : n_cu), dim3(kPipeThreads), kPipeLds,
                       (hipStream_t)stream, (const uint8_t*)x8, (const uint8_t*)w8, T, D, I, scale, wscale, amax,
                       (uint8_t*)gu8, (uint8_t*)h8, (uint8_t*)h8t, ldt, tiles_m, tiles_n, (const int*)nullptr,
                       (int64_t)0);
    return status();
  }
  const int tiles_m = cdiv(T, kTile), tiles_n = (int)(I / 128);
  int rc = prep(swiglu_fwd_kernel, kMainLds);
  if (rc) return rc;
  hipLaunchKernelGGL(swiglu_fwd_kernel, dim3(tiles_m * tiles_n), dim3(512), kMainLds, (hipStream_t)stream,
                     (const uint8_t*)x8, (const uint8_t*)w8, T, D, I, scale, wscale, amax, (uint8_t*)gu8,
                     (uint8_t*)h8, (uint8_t*)h8t, ldt, tiles_m, tiles_n, (const int*)nullptr, (int64_t)0);
  return status();
}

int sfp8_gemm_down_fwd(const void* h8, const void* wd8, const void* res, int64_t T, int64_t D, int64_t I,
                       const float* scale, const float* wscale, void* y, int64_t ldt, void* stream) {
  if (!wd8 || !scale || !wscale || (T > 0 && (!h8 || !res || !y))) return kErrNullPointer;
  if (T < 0 || D <= 0 || I <= 0 || I % (2 * kStage) || D % 16 || ldt < T || ldt % kTile) return kErrBadShape;
  if (!fits32(ldt, I) || !fits32(slab_rows(D), I) || !fits32(kTile, 2 * D)) return kErrBadShape;
  if (!al16(h8) || !al16(wd8) || !al16(res) || !al16(y)) return kErrBadAlignment;
  if (T == 0) return kOk;
  const int tiles_m = cdiv(T, kTile), tiles_n = cdiv(D, kTile);
  int rc = prep(down_fwd_kernel, kMainLds);
  if (rc) return rc;
  hipLaunchKernelGGL(down_fwd_kernel, dim3(tiles_m * tiles_n), dim3(512), kMainLds, (hipStream_t)stream,
                     (const uint8_t*)h8, (const uint8_t*)wd8, (const uint16_t*)res, T, D, I, scale, wscale + 1,
                     (uint16_t*)y, ldt, tiles_m, tiles_n, (const int*)nullptr, (int64_t)0);
  return status();
}

int sfp8_gemm_down_dgrad_swiglu(const void* dy, const void* wdt, const void* gu8, int64_t T, int64_t D,
                                int64_t I, const float* scale, float* amax, void* dgu8, void* dgu8t,
                                int64_t ldt, void* stream) {
  if (!wdt || !scale || !amax || (T > 0 && (!dy || !gu8 || !dgu8))) return kErrNullPointer;
  if (T < 0 || D <= 0 || I <= 0 || (2 * D) % (2 * kStage) || I % 128 || ldt != (int64_t)cdiv(T, kTile) * kTile)
    return kErrBadShape;  // ldt = T rounded up to 256: the grid writes every padding token
  if (!fits32(kTile, 2 * D) || !fits32(slab_rows(I), 2 * D) || !fits32(ldt, 2 * I)) return kErrBadShape;
  if (!al16(dy) || !al16(wdt) || !al16(gu8) || !al16(dgu8) || !al16(dgu8t)) return kErrBadAlignment;
  if (T == 0) return kOk;
  const int tiles_m = cdiv(T, kTile), tiles_n = cdiv(I, kTile);
  const int ntiles = tiles_m * tiles_n;
  int n_cu = 0;
  int rc = cu_count(&n_cu);
  if (rc) return rc;
  const int grid = ntiles < n_cu ? ntiles : n_cu;
  const auto kern = dgu8t ? down_dgrad_swiglu_kernel<true> : down_dgrad_swiglu_kernel<false>;
  rc = prep(kern, kDgradLds);
  if (rc) return rc;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(512), kDgradLds, (hipStream_t)stream,
                     (const uint16_t*)dy, (const uint16_t*)wdt, (const uint8_t*)gu8, T, D, I, scale, amax,
                     (uint8_t*)dgu8, (uint8_t*)dgu8t, ldt, tiles_m, tiles_n, (const int*)nullptr, (int64_t)0);
  return status();
}

int sfp8_gemm_gateup_dgrad(const void* dgu8, const void* w8t, int64_t T, int64_t D, int64_t I,
                           const float* scale, const float* wscale, void* dxn, int64_t ldt, void* stream) {
  if (!w8t || !scale || !wscale || (T > 0 && (!dgu8 || !dxn))) return kErrNullPointer;
  if (T < 0 || D <= 0 || I <= 0 || (2 * I) % (2 * kStage) || D % 16 || ldt < T || ldt % kTile) return kErrBadShape;
  if (!fits32(ldt, 2 * I) || !fits32(slab_rows(D), 2 * I) || !fits32(kTile, 2 * D)) return kErrBadShape;
  if (!al16(dgu8) || !al16(w8t) || !al16(dxn)) return kErrBadAlignment;
  if (T == 0) return kOk;
  const int tiles_m = cdiv(T, kTile), tiles_n = cdiv(D, kTile);
  int rc = prep(gateup_dgrad_kernel, kMainLds);
  if (rc) return rc;
  hipLaunchKernelGGL(gateup_dgrad_kernel, dim3(tiles_m * tiles_n), dim3(512), kMainLds, (hipStream_t)stream,
                     (const uint8_t*)dgu8, (const uint8_t*)w8t, T, D, I, scale, wscale, (uint16_t*)dxn, ldt,
                     tiles_m, tiles_n, (const int*)nullptr, (int64_t)0);
  return status();
}

// Number of K splits the library uses for an (M, N, ldt) weight gradient and
// the workspace (floats) it needs: splits * M * N when splits > 1, else 0.
// Split sp covers K [sp * c, min((sp + 1) * c, ldt)) with c = wgrad_chunk:
// ldt / s rounded up to whole 128-token (128-byte) stage pairs, so the last
// split may be shorter.  s is usable when every split has at least 2048
// tokens' worth of chunk and the last split is not empty.
static bool wgrad_split_ok(int64_t s, int64_t ldt) {
  if (s == 1) return true;
  const int64_t c = wgrad_chunk(ldt, s);
  return c >= 2048 && ldt - (s - 1) * c > 0;
}

// bf16 operands (ldt counts K bytes): splits double while the grid has fewer
// than 512 work-groups, stopping at 8 once it has 384; every split equal.
static int64_t wgrad_splits_doubling(int64_t M, int64_t N, int64_t ldt) {
  const int64_t tiles = (int64_t)cdiv(M, kTile) * cdiv(N, kTile);
  int64_t s = 1;
  while (tiles * s < 512 && !(s >= 8 && tiles * s >= 384) && ldt % (2 * s) == 0 &&
         (ldt / (2 * s)) % (2 * kStage) == 0 && ldt / (2 * s) >= 2048)
    s *= 2;
  return s;
}

int64_t sfp8_wgrad_splits(int64_t M, int64_t N, int64_t ldt) {
  // The count (any, not only a power of two) that minimises the modelled
  // time: the rounds of work-groups the 256 CUs run, times the longest
  // split's 64-token K stages, plus the split partials' traffic (4 bytes
  // written and read per output and split, at about 5 TB/s: M * N * 8 /
  // 3.5e6 stage times of 0.7 us).  At T = 65536 this gives 5 splits for both
  // the down gradient (48 tiles: 240 work-groups in one round, where 4
  // splits leave 64 CUs idle) and the gate/up one (96 tiles: 480 work-groups
  // in two rounds, against three rounds of 256 with 8).  Ties go to fewer
  // splits.
  constexpr int64_t kCUs = 256;
  const int64_t tiles = (int64_t)cdiv(M, kTile) * cdiv(N, kTile);
  const double part = (double)M * (double)N * 8.0 / 3.5e6;
  int64_t best = 1;
  double best_cost = 0.0;
  for (int64_t s = 1; s <= 64 && tiles * s <= 2048; ++s) {
    if (!wgrad_split_ok(s, ldt)) continue;
    const double stages = (double)wgrad_chunk(ldt, s) / kStage;
    const double cost = (double)((tiles * s + kCUs - 1) / kCUs) * stages + (s > 1 ? s * part : 0.0);
    if (s == 1 || cost < best_cost - 1e-9) {
      best = s;
      best_cost = cost;
    }
  }
  return best;
}

int64_t sfp8_slab_bytes(int64_t rows, int64_t k) {
  if (rows < 0 || k < 0 || k % kStage) return -1;
  return slab_rows(rows) * k;
}

int64_t sfp8_wgrad_workspace_floats(int64_t M, int64_t N, int64_t ldt) {
  // one 256 x 256 fp32 tile per (split, tile)
  const int64_t s = sfp8_wgrad_splits(M, N, ldt);
  return s > 1 ? s * (int64_t)cdiv(M, kTile) * cdiv(N, kTile) * kTile * kTile : 0;
}



int sfp8_gemm_wgrad(const void* at, int fmt_a, const void* bt, int fmt_b, int64_t M, int64_t N, int64_t ldt,
                    const float* sa, const float* sb, float* out, float* ws, int64_t ws_floats, void* stream) {
  if (!sa || !sb || !out || (ldt > 0 && (!at || !bt))) return kErrNullPointer;
  if (M <= 0 || N <= 0 || ldt < 0 || ldt % kTile || N % 4) return kErrBadShape;
  if (fmt_a != kFmtE5M2 || fmt_b != kFmtE4M3) return kErrBadShape;
  // every K-slab offset (stage * rows * 64 + row * 64) is 32-bit
  if (!fits32(slab_rows(M), ldt) || !fits32(slab_rows(N), ldt)) return kErrBadShape;
  if (!al16(at) || !al16(bt) || !al16(out)) return kErrBadAlignment;
  hipStream_t st = (hipStream_t)stream;
  const int64_t splits = sfp8_wgrad_splits(M, N, ldt);
  if (splits > 1 && (!ws || ws_floats < sfp8_wgrad_workspace_floats(M, N, ldt))) return kErrWorkspaceTooSmall;
  if (ldt == 0) {
    // no tokens: the gradient is zero (a fill kernel, not a memset node, so
    // that a captured graph replays it correctly)
    const int64_t n = M * N;
    hipLaunchKernelGGL(zero_fill_kernel, dim3((unsigned)((n + 1023) / 1024)), dim3(256), 0, st, out, n);
    return status();
  }
  const int tiles_m = cdiv(M, kTile), tiles_n = cdiv(N, kTile);
  int rc = prep(wgrad_kernel<false, kFmtE5M2, kFmtE4M3, false, false, kWgradWaves>, kMainLds);
  if (rc) return rc;
  hipLaunchKernelGGL((wgrad_kernel<false, kFmtE5M2, kFmtE4M3, false, false, kWgradWaves>),
                     dim3((unsigned)wgrad_grid(tiles_m * tiles_n, (int)splits)), dim3(64 * kWgradWaves), kMainLds, st,
                     (const uint8_t*)at, (const uint8_t*)bt, M, N, ldt, wgrad_chunk(ldt, splits), sa, sb,
                     splits > 1 ? ws : out, tiles_m, tiles_n, (int)splits, (int)(splits > 1), TrOp{}, TrOp{});
  rc = status();
  if (rc || splits == 1) return rc;
  const int64_t n4 = (int64_t)tiles_m * tiles_n * kTile * kTile / 4;
  hipLaunchKernelGGL((splitk_reduce_kernel<false, kWgradWaves>), dim3((unsigned)((n4 + 255) / 256), 1), dim3(256), 0,
                     st, ws, (int)splits, n4, tiles_n, M, N, sa, sb, out);
  return status();
}

// ---- grouped (MoE expert) GEMMs over padded expert order (common.h) ----
// ldp = padded rows (256 * sfp8_moe_padded_rows); plan from sfp8_moe_plan.
namespace {
inline bool moe_shape(int64_t E, int64_t D, int64_t I, int64_t ldp) {
  return E > 0 && D > 0 && I > 0 && D % 128 == 0 && I % 128 == 0 && ldp > 0 && ldp % kTile == 0;
}
}  // namespace

int sfp8_moe_gemm_gateup_swiglu_fwd(const void* x8, const void* w8, int64_t E, int64_t D, int64_t I, const int* plan,
                                    int64_t ldp, const float* scale, const float* q_gu, float* amax, void* gu8,
                                    void* h8, void* h8t, void* stream) {
  if (!x8 || !w8 || !plan || !scale || !q_gu || !amax || !gu8 || !h8) return kErrNullPointer;
  if (!moe_shape(E, D, I, ldp) || !fits32(ldp, D) || !fits32(2 * I, D) || !fits32(ldp, 2 * I)) return kErrBadShape;
  if (!al16(x8) || !al16(w8) || !al16(gu8) || !al16(h8) || !al16(h8t)) return kErrBadAlignment;
  if (D == 1024) {
    // the persistent kernel walks the plan's tiles (its count read on the
    // device); the grid is sized for the worst case
    const int tiles_m = (int)(ldp / kTile), tiles_n = (int)(I / 64);
    const int ntiles = tiles_m * tiles_n;
    int n_cu = 0;
    int rc = cu_count(&n_cu);
    if (rc) return rc;
    rc = prep(swiglu_pipe_kernel<16, kPipeTB>, kPipeLds);
    if (rc) return rc;
    hipLaunchKernelGGL((swiglu_pipe_kernel<16, kPipeTB>), dim3(ntiles < n_cu ? ntiles : n_cu), dim3(kPipeThreads), kPipeLds,
                       (hipStream_t)stream, (const uint8_t*)x8, (const uint8_t*)w8, ldp, D, I, scale, q_gu, amax,
                       (uint8_t*)gu8, (uint8_t*)h8, (uint8_t*)h8t, ldp, tiles_m, tiles_n, plan,
                       D * slab_rows(2 * I));
    return status();
  }
  const int tiles_m = (int)(ldp / kTile), tiles_n = (int)(I / 128);
  int rc = prep(swiglu_fwd_kernel, kMainLds);
  if (rc) return rc;
  hipLaunchKernelGGL(swiglu_fwd_kernel, dim3(tiles_m * tiles_n), dim3(512), kMainLds, (hipStream_t)stream,
                     (const uint8_t*)x8, (const uint8_t*)w8, ldp, D, I, scale, q_gu, amax, (uint8_t*)gu8,
                     (uint8_t*)h8, (uint8_t*)h8t, ldp, tiles_m, tiles_n, plan, D * slab_rows(2 * I));
  return status();
}

int sfp8_moe_gemm_down_fwd(const void* h8, const void* wd8, int64_t E, int64_t D, int64_t I, const int* plan,
                           int64_t ldp, const float* scale, const float* q_d, void* out, int64_t R, void* stream) {
  if (!h8 || !wd8 || !plan || !scale || !q_d || (R > 0 && !out)) return kErrNullPointer;
  if (!moe_shape(E, D, I, ldp) || R < 0 || !fits32(ldp, I) || !fits32(slab_rows(D), I) || !fits32(kTile, 2 * D))
    return kErrBadShape;
  if (!al16(h8) || !al16(wd8) || !al16(out)) return kErrBadAlignment;
  const int tiles_m = (int)(ldp / kTile), tiles_n = cdiv(D, kTile);
  int rc = prep(down_fwd_kernel, kMainLds);
  if (rc) return rc;
  hipLaunchKernelGGL(down_fwd_kernel, dim3(tiles_m * tiles_n), dim3(512), kMainLds, (hipStream_t)stream,
                     (const uint8_t*)h8, (const uint8_t*)wd8, (const uint16_t*)nullptr, R, D, I, scale, q_d,
                     (uint16_t*)out, ldp, tiles_m, tiles_n, plan, I * slab_rows(D));
  return status();
}

int sfp8_moe_gemm_down_dgrad_swiglu(const void* dout, const void* wdt, const void* gu8, int64_t E, int64_t D,
                                    int64_t I, int64_t R, const int* plan, int64_t ldp, const float* scale,
                                    float* amax, void* dgu8, void* dgu8t, void* stream) {
  if (!wdt || !gu8 || !plan || !scale || !amax || !dgu8 || (R > 0 && !dout)) return kErrNullPointer;
  if (!moe_shape(E, D, I, ldp) || R < 0) return kErrBadShape;
  if (!fits32(kTile, 2 * D) || !fits32(slab_rows(I), 2 * D) || !fits32(ldp, 2 * I)) return kErrBadShape;
  if (!al16(dout) || !al16(wdt) || !al16(gu8) || !al16(dgu8) || !al16(dgu8t)) return kErrBadAlignment;
  int n_cu = 0;
  int rc = cu_count(&n_cu);
  if (rc) return rc;
  const int tiles_m = (int)(ldp / kTile), tiles_n = cdiv(I, kTile);
  const int ntiles = tiles_m * tiles_n;  // an upper bound: the kernel reads the plan's count
  const auto kern = dgu8t ? down_dgrad_swiglu_kernel<true> : down_dgrad_swiglu_kernel<false>;
  rc = prep(kern, kDgradLds);
  if (rc) return rc;
  hipLaunchKernelGGL(kern, dim3(ntiles < n_cu ? ntiles : n_cu), dim3(512), kDgradLds,
                     (hipStream_t)stream, (const uint16_t*)dout, (const uint16_t*)wdt, (const uint8_t*)gu8, R, D, I,
                     scale, amax, (uint8_t*)dgu8, (uint8_t*)dgu8t, ldp, tiles_m, tiles_n, plan,
                     2 * D * slab_rows(I));
  return status();
}

int sfp8_moe_gemm_gateup_dgrad(const void* dgu8, const void* w8t, int64_t E, int64_t D, int64_t I, const int* plan,
                               int64_t ldp, const float* scale, const float* q_gu, void* dx, int64_t R, void* stream) {
  if (!dgu8 || !w8t || !plan || !scale || !q_gu || (R > 0 && !dx)) return kErrNullPointer;
  if (!moe_shape(E, D, I, ldp) || R < 0 || !fits32(ldp, 2 * I) || !fits32(slab_rows(D), 2 * I) ||
      !fits32(kTile, 2 * D))
    return kErrBadShape;
  if (!al16(dgu8) || !al16(w8t) || !al16(dx)) return kErrBadAlignment;
  const int tiles_m = (int)(ldp / kTile), tiles_n = cdiv(D, kTile);
  int rc = prep(gateup_dgrad_kernel, kMainLds);
  if (rc) return rc;
  hipLaunchKernelGGL(gateup_dgrad_kernel, dim3(tiles_m * tiles_n), dim3(512), kMainLds, (hipStream_t)stream,
                     (const uint8_t*)dgu8, (const uint8_t*)w8t, R, D, I, scale, q_gu, (uint16_t*)dx, ldp, tiles_m,
                     tiles_n, plan, 2 * I * slab_rows(D));
  return status();
}

// K splits of a grouped weight gradient: enough work-groups to fill the GPU
// (about 512) when there are few experts and tiles.
int64_t sfp8_moe_wgrad_splits(int64_t M, int64_t N, int64_t E) {
  // at least 2 splits, then doubling until the grid has 384 work-groups (8 at
  // most): at the MoE headline shape (8 experts, D=1024, I=1536) the down
  // gradient takes 0.234 ms with 2 splits against 0.245 with 4, the gate/up
  // one 0.397 with 2 against 0.413 with 1
  const int64_t wgs = (int64_t)cdiv(M, kTile) * cdiv(N, kTile) * E;
  int64_t s = 1;
  while (s < 8 && (s < 2 || wgs * s < 384)) s *= 2;
  return s;
}

int64_t sfp8_moe_wgrad_workspace_floats(int64_t M, int64_t N, int64_t E) {
  const int64_t s = sfp8_moe_wgrad_splits(M, N, E);
  return s > 1 ? E * s * (int64_t)cdiv(M, kTile) * cdiv(N, kTile) * kTile * kTile : 0;
}

int sfp8_moe_gemm_wgrad(const void* at, int fmt_a, const void* bt, int fmt_b, int64_t M, int64_t N, int64_t E,
                        const int* plan, int64_t ldp, const float* sa, const float* sb, float* out, float* ws,
                        int64_t ws_floats, void* stream) {
  if (!at || !bt || !plan || !sa || !sb || !out) return kErrNullPointer;
  if (M <= 0 || N <= 0 || E <= 0 || N % 4 || ldp <= 0 || ldp % kTile) return kErrBadShape;
  if (fmt_a != kFmtE5M2 || fmt_b != kFmtE4M3) return kErrBadShape;
  if (!fits32(slab_rows(M), ldp) || !fits32(slab_rows(N), ldp)) return kErrBadShape;
  if (!al16(at) || !al16(bt) || !al16(out) || !al16(ws)) return kErrBadAlignment;
  const int64_t splits = sfp8_moe_wgrad_splits(M, N, E);
  if (splits > 1 && (!ws || ws_floats < sfp8_moe_wgrad_workspace_floats(M, N, E))) return kErrWorkspaceTooSmall;
  hipStream_t st = (hipStream_t)stream;
  const int tiles_m = cdiv(M, kTile), tiles_n = cdiv(N, kTile);
  int rc = prep(moe_wgrad_kernel<false, kFmtE5M2, kFmtE4M3, false, false, kWgradWaves>, kMainLds);
  if (rc) return rc;
  hipLaunchKernelGGL((moe_wgrad_kernel<false, kFmtE5M2, kFmtE4M3, false, false, kWgradWaves>),
                     dim3((unsigned)(tiles_m * tiles_n * splits * E)), dim3(64 * kWgradWaves), kMainLds, st,
                     (const uint8_t*)at, (const uint8_t*)bt, M, N, ldp, sa, sb, out, ws, plan, tiles_m, tiles_n,
                     (int)splits);
  rc = status();
  if (rc || splits == 1) return rc;
  const int64_t n4 = (int64_t)tiles_m * tiles_n * kTile * kTile / 4;
  hipLaunchKernelGGL((splitk_reduce_kernel<false, kWgradWaves>), dim3((unsigned)((n4 + 255) / 256), (unsigned)E),
                     dim3(256), 0, st, ws, (int)splits, n4, tiles_n, M, N, sa, sb, out);
  return status();
}

// ---- the grouped weight gradient with row K-slab operands ----
int64_t sfp8_moe_wgrad_rows_workspace_floats(int64_t M, int64_t N, int64_t E) {
  return E * sfp8_moe_wgrad_splits(M, N, E) * (int64_t)cdiv(M, kTile) * cdiv(N, kTile) * kTile * kTile;
}

int sfp8_moe_gemm_wgrad_rows(const void* a, int fmt_a, int a_rows, const void* b, int fmt_b, int b_rows, int64_t M,
                             int64_t N, int64_t E, const int* plan, int64_t ldp, const float* sa, const float* sb,
                             float* out, float* ws, int64_t ws_floats, void* stream) {
  if (!a || !b || !plan || !sa || !sb || !out || !ws) return kErrNullPointer;
  if (M <= 0 || N <= 0 || E <= 0 || N % 4 || ldp <= 0 || ldp % kTile || !(a_rows || b_rows)) return kErrBadShape;
  if ((a_rows && M % 64) || (b_rows && N % 64)) return kErrBadShape;
  if (fmt_a != kFmtE5M2 || fmt_b != kFmtE4M3) return kErrBadShape;
  if (!fits32(slab_rows(M), ldp) || !fits32(slab_rows(N), ldp)) return kErrBadShape;
  if (!al16(a) || !al16(b) || !al16(out) || !al16(ws)) return kErrBadAlignment;
  const int64_t splits = sfp8_moe_wgrad_splits(M, N, E);
  if (ws_floats < sfp8_moe_wgrad_rows_workspace_floats(M, N, E)) return kErrWorkspaceTooSmall;
  hipStream_t st = (hipStream_t)stream;
  const int tiles_m = cdiv(M, kTile), tiles_n = cdiv(N, kTile);
  const dim3 grid((unsigned)(tiles_m * tiles_n * splits * E));
  int rc;
  if (a_rows && b_rows) {
    rc = prep(moe_wgrad_kernel<false, kFmtE5M2, kFmtE4M3, true, true, kWgradWaves>, kMainLds);
    if (!rc)
      hipLaunchKernelGGL((moe_wgrad_kernel<false, kFmtE5M2, kFmtE4M3, true, true, kWgradWaves>), grid,
                         dim3(64 * kWgradWaves), kMainLds, st,
                         (const uint8_t*)a, (const uint8_t*)b, M, N, ldp, sa, sb, out, ws, plan, tiles_m, tiles_n,
                         (int)splits);
  } else if (a_rows) {
    rc = prep(moe_wgrad_kernel<false, kFmtE5M2, kFmtE4M3, true, false, kWgradWaves>, kMainLds);
    if (!rc)
      hipLaunchKernelGGL((moe_wgrad_kernel<false, kFmtE5M2, kFmtE4M3, true, false, kWgradWaves>), grid,
                         dim3(64 * kWgradWaves), kMainLds, st,
                         (const uint8_t*)a, (const uint8_t*)b, M, N, ldp, sa, sb, out, ws, plan, tiles_m, tiles_n,
                         (int)splits);
  } else {
    rc = prep(moe_wgrad_kernel<false, kFmtE5M2, kFmtE4M3, false, true, kWgradWaves>, kMainLds);
    if (!rc)
      hipLaunchKernelGGL((moe_wgrad_kernel<false, kFmtE5M2, kFmtE4M3, false, true, kWgradWaves>), grid,
                         dim3(64 * kWgradWaves), kMainLds, st,
                         (const uint8_t*)a, (const uint8_t*)b, M, N, ldp, sa, sb, out, ws, plan, tiles_m, tiles_n,
                         (int)splits);
  }
  if (rc) return rc;
  rc = status();
  if (rc) return rc;
  const int64_t n4 = (int64_t)tiles_m * tiles_n * kTile * kTile / 4;
  if (b_rows)
    hipLaunchKernelGGL((splitk_reduce_kernel<true, kWgradWaves>), dim3((unsigned)((n4 + 255) / 256), (unsigned)E),
                       dim3(256), 0, st, ws, (int)splits, n4, tiles_n, M, N, sa, sb, out);
  else
    hipLaunchKernelGGL((splitk_reduce_kernel<false, kWgradWaves>), dim3((unsigned)((n4 + 255) / 256), (unsigned)E),
                       dim3(256), 0, st, ws, (int)splits, n4, tiles_n, M, N, sa, sb, out);
  return status();
}


// ---- bf16 SwiGLU path (the default, non-FP8 path) ----
namespace {
// (a tile's gu rows, 256 x 2I bf16, are addressed with 32-bit offsets)
inline bool bf16_shape(int64_t D, int64_t I) {
  return D > 0 && I > 0 && D % 64 == 0 && I % 64 == 0 && fits32(kTile, 4 * I);
}

int bf16_swiglu_launch(const void* x, const void* w, int64_t T, int64_t D, int64_t I, const float* rstd, void* gu,
                       void* h, const int* plan, int64_t E, int tiles_m, int64_t ldxs, hipStream_t st) {
  const int tiles_n = cdiv(I, 128);
  int rc = prep(bf16_swiglu_fwd_kernel, kMainLds);
  if (rc) return rc;
  hipLaunchKernelGGL(bf16_swiglu_fwd_kernel, dim3((unsigned)(tiles_m * tiles_n)), dim3(512), kMainLds, st,
                     (const uint16_t*)x, (const uint8_t*)w, T, D, I, rstd, (uint16_t*)gu, (uint16_t*)h, tiles_m,
                     tiles_n, plan, plan ? 2 * D * slab_rows(2 * I) : 0, ldxs);
  (void)E;
  return status();
}

int bf16_gemm_launch(const void* a, const void* b, int64_t T, int64_t N, int64_t K, int64_t lda, void* out,
                     const int* plan, int tiles_m, hipStream_t st) {
  const int tiles_n = cdiv(N, kTile);
  int rc = prep(bf16_gemm_kernel, kMainLds);
  if (rc) return rc;
  hipLaunchKernelGGL(bf16_gemm_kernel, dim3((unsigned)(tiles_m * tiles_n)), dim3(512), kMainLds, st,
                     (const uint8_t*)a, (const uint8_t*)b, T, N, 2 * K, lda, (uint16_t*)out, tiles_m, tiles_n, plan,
                     plan ? 2 * K * slab_rows(N) : 0);
  return status();
}
}  // namespace

int sfp8_bf16_gemm_swiglu_fwd(const void* x, int x_slab, const void* w, int64_t T, int64_t D, int64_t I,
                              const float* rstd, void* gu, void* h, void* stream) {
  if (!w || (T > 0 && (!x || !gu || !h))) return kErrNullPointer;
  if (T < 0 || !bf16_shape(D, I) || !fits32(kTile, 2 * D) || !fits32(slab_rows(2 * I), 2 * D)) return kErrBadShape;
  if (x_slab && !fits32(slab_rows(T), 2 * D)) return kErrBadShape;
  if (!al16(x) || !al16(w) || !al16(gu) || !al16(h)) return kErrBadAlignment;
  if (T == 0) return kOk;
  return bf16_swiglu_launch(x, w, T, D, I, rstd, gu, h, nullptr, 1, cdiv(T, kTile), x_slab ? slab_rows(T) : 0,
                            (hipStream_t)stream);
}

int sfp8_bf16_moe_gemm_swiglu_fwd(const void* x, const void* w, int64_t E, int64_t D, int64_t I, const int* plan,
                                  int64_t ldp, void* gu, void* h, void* stream) {
  if (!w || !plan || (ldp > 0 && (!x || !gu || !h))) return kErrNullPointer;
  if (E <= 0 || ldp < 0 || ldp % kTile || !bf16_shape(D, I) || !fits32(kTile, 2 * D) ||
      !fits32(slab_rows(2 * I), 2 * D))
    return kErrBadShape;
  if (!al16(x) || !al16(w) || !al16(gu) || !al16(h)) return kErrBadAlignment;
  if (ldp == 0) return kOk;
  return bf16_swiglu_launch(x, w, 0, D, I, nullptr, gu, h, plan, E, (int)(ldp / kTile), 0, (hipStream_t)stream);
}

int sfp8_bf16_gemm(const void* a, const void* b, int64_t T, int64_t N, int64_t K, int64_t lda, void* out,
                   void* stream) {
  if (!b || (T > 0 && (!a || !out))) return kErrNullPointer;
  if (T < 0 || N <= 0 || N % 8 || K <= 0 || K % 32 || lda < T || lda % kTile) return kErrBadShape;
  if (!fits32(lda, 2 * K) || !fits32(slab_rows(N), 2 * K) || !fits32(kTile, 2 * N)) return kErrBadShape;
  if (!al16(a) || !al16(b) || !al16(out)) return kErrBadAlignment;
  if (T == 0) return kOk;
  return bf16_gemm_launch(a, b, T, N, K, lda, out, nullptr, cdiv(T, kTile), (hipStream_t)stream);
}

int sfp8_bf16_moe_gemm(const void* a, const void* b, int64_t E, int64_t N, int64_t K, const int* plan, int64_t ldp,
                       void* out, void* stream) {
  if (!b || !plan || (ldp > 0 && (!a || !out))) return kErrNullPointer;
  if (E <= 0 || N <= 0 || N % 8 || K <= 0 || K % 32 || ldp < 0 || ldp % kTile) return kErrBadShape;
  if (!fits32(ldp, 2 * K) || !fits32(slab_rows(N), 2 * K)) return kErrBadShape;
  if (!al16(a) || !al16(b) || !al16(out)) return kErrBadAlignment;
  if (ldp == 0) return kOk;
  return bf16_gemm_launch(a, b, 0, N, K, ldp, out, plan, (int)(ldp / kTile), (hipStream_t)stream);
}

int64_t sfp8_bf16_wgrad_splits(int64_t M, int64_t N, int64_t ldt) { return wgrad_splits_doubling(M, N, 2 * ldt); }

int64_t sfp8_bf16_wgrad_workspace_floats(int64_t M, int64_t N, int64_t ldt) {
  return sfp8_bf16_wgrad_splits(M, N, ldt) * (int64_t)cdiv(M, kTile) * cdiv(N, kTile) * kTile * kTile;
}

int sfp8_bf16_gemm_wgrad(const void* at, const void* bt, int64_t M, int64_t N, int64_t ldt, void* out, float* ws,
                         int64_t ws_floats, void* stream) {
  if (!out || (ldt > 0 && (!at || !bt))) return kErrNullPointer;
  if (M <= 0 || N <= 0 || ldt < 0 || ldt % kTile || N % 4 || (M * N) % 8) return kErrBadShape;
  if (!fits32(slab_rows(M), 2 * ldt) || !fits32(slab_rows(N), 2 * ldt)) return kErrBadShape;
  if (!al16(at) || !al16(bt) || !al16(out) || !al16(ws)) return kErrBadAlignment;
  hipStream_t st = (hipStream_t)stream;
  if (ldt == 0) {
    // no tokens: a zero gradient (M * N bf16 = M * N / 2 floats of zero bits)
    const int64_t n = M * N / 2;
    hipLaunchKernelGGL(zero_fill_kernel, dim3((unsigned)((n + 1023) / 1024)), dim3(256), 0, st, (float*)out, n);
    return status();
  }
  const int64_t splits = sfp8_bf16_wgrad_splits(M, N, ldt);
  if (!ws || ws_floats < sfp8_bf16_wgrad_workspace_floats(M, N, ldt)) return kErrWorkspaceTooSmall;
  const int tiles_m = cdiv(M, kTile), tiles_n = cdiv(N, kTile);
  int rc = prep(wgrad_kernel<true, 0, 0, false, false, kBf16WgradWaves>, kMainLds);
  if (rc) return rc;
  hipLaunchKernelGGL((wgrad_kernel<true, 0, 0, false, false, kBf16WgradWaves>), dim3((unsigned)(tiles_m * tiles_n * splits)),
                     dim3(64 * kBf16WgradWaves), kMainLds, st, (const uint8_t*)at, (const uint8_t*)bt, M, N, 2 * ldt,
                     2 * ldt / splits, nullptr, nullptr, ws, tiles_m, tiles_n, (int)splits, 1, TrOp{}, TrOp{});
  rc = status();
  if (rc) return rc;
  const int64_t n4 = (int64_t)tiles_m * tiles_n * kTile * kTile / 4;
  hipLaunchKernelGGL((bf16_wgrad_reduce_kernel<false, kBf16WgradWaves>), dim3((unsigned)((n4 + 255) / 256), 1), dim3(256),
                     0, st, ws, (int)splits, n4, tiles_n, M, N, (uint16_t*)out);
  return status();
}

int64_t sfp8_bf16_moe_wgrad_workspace_floats(int64_t M, int64_t N, int64_t E) {
  return E * sfp8_moe_wgrad_splits(M, N, E) * (int64_t)cdiv(M, kTile) * cdiv(N, kTile) * kTile * kTile;
}

int sfp8_bf16_moe_gemm_wgrad(const void* at, const void* bt, int64_t M, int64_t N, int64_t E, const int* plan,
                             int64_t ldp, void* out, float* ws, int64_t ws_floats, void* stream) {
  if (!at || !bt || !plan || !out) return kErrNullPointer;
  if (M <= 0 || N <= 0 || E <= 0 || N % 4 || ldp <= 0 || ldp % kTile) return kErrBadShape;
  if (!fits32(slab_rows(M), 2 * ldp) || !fits32(slab_rows(N), 2 * ldp)) return kErrBadShape;
  if (!al16(at) || !al16(bt) || !al16(out) || !al16(ws)) return kErrBadAlignment;
  const int64_t splits = sfp8_moe_wgrad_splits(M, N, E);
  if (!ws || ws_floats < sfp8_bf16_moe_wgrad_workspace_floats(M, N, E)) return kErrWorkspaceTooSmall;
  hipStream_t st = (hipStream_t)stream;
  const int tiles_m = cdiv(M, kTile), tiles_n = cdiv(N, kTile);
  int rc = prep(moe_wgrad_kernel<true, 0, 0, false, false, kBf16WgradWaves>, kMainLds);
  if (rc) return rc;
  hipLaunchKernelGGL((moe_wgrad_kernel<true, 0, 0, false, false, kBf16WgradWaves>),
                     dim3((unsigned)(tiles_m * tiles_n * splits * E)), dim3(64 * kBf16WgradWaves), kMainLds, st,
                     (const uint8_t*)at, (const uint8_t*)bt, M, N, 2 * ldp, nullptr, nullptr, nullptr, ws, plan,
                     tiles_m, tiles_n, (int)splits);
  rc = status();
  if (rc) return rc;
  const int64_t n4 = (int64_t)tiles_m * tiles_n * kTile * kTile / 4;
  hipLaunchKernelGGL((bf16_wgrad_reduce_kernel<false, kBf16WgradWaves>), dim3((unsigned)((n4 + 255) / 256), (unsigned)E),
                     dim3(256), 0, st, ws, (int)splits, n4, tiles_n, M, N, (uint16_t*)out);
  return status();
}

// ---- the bf16 weight gradients read through transposing LDS reads ----
int sfp8_bf16_gemm_wgrad_rows(const void* a, const void* x, int x_rows, int64_t M, int64_t N, int64_t T, int64_t ldt,
                              void* out, float* ws, int64_t ws_floats, void* stream) {
  if (!out || (T > 0 && (!a || !x))) return kErrNullPointer;
  if (M <= 0 || N <= 0 || M % 32 || N % (x_rows ? 32 : 4) || T < 0 || ldt < T || ldt % kTile || (M * N) % 8)
    return kErrBadShape;
  if (!fits32(slab_rows(M), 2 * ldt) || !fits32(slab_rows(N), 2 * ldt) || T * N * 2 >= ((int64_t)1 << 31))
    return kErrBadShape;
  if (!al16(a) || !al16(x) || !al16(out) || !al16(ws)) return kErrBadAlignment;
  hipStream_t st = (hipStream_t)stream;
  if (ldt == 0) {
    const int64_t n = M * N / 2;
    hipLaunchKernelGGL(zero_fill_kernel, dim3((unsigned)((n + 1023) / 1024)), dim3(256), 0, st, (float*)out, n);
    return status();
  }
  const int64_t splits = sfp8_bf16_wgrad_splits(M, N, ldt);
  if (!ws || ws_floats < sfp8_bf16_wgrad_workspace_floats(M, N, ldt)) return kErrWorkspaceTooSmall;
  const int tiles_m = cdiv(M, kTile), tiles_n = cdiv(N, kTile);
  // a: the bf16 K-slab of [ldt, M] (32 columns per 64-byte row); x (x_rows):
  // row-major [T, N] bf16, tokens T..ldt-1 read as zero through the range
  // check, or else the token-contiguous bf16 K-slab of x^T over ldt tokens
  const TrOp tra{kStage, ldt * kStage, (M / 32) * ldt * kStage}, trb{2 * N, kStage, T * 2 * N};
  const dim3 grid((unsigned)(tiles_m * tiles_n * splits));
  int rc;
  if (x_rows) {
    rc = prep(wgrad_kernel<true, 0, 0, true, true, kBf16WgradWaves>, kMainLds);
    if (!rc)
      hipLaunchKernelGGL((wgrad_kernel<true, 0, 0, true, true, kBf16WgradWaves>), grid, dim3(64 * kBf16WgradWaves),
                         kMainLds, st, (const uint8_t*)a, (const uint8_t*)x, M, N, 2 * ldt, 2 * ldt / splits, nullptr,
                         nullptr, ws, tiles_m, tiles_n, (int)splits, 1, tra, trb);
  } else {
    rc = prep(wgrad_kernel<true, 0, 0, true, false, kBf16WgradWaves>, kMainLds);
    if (!rc)
      hipLaunchKernelGGL((wgrad_kernel<true, 0, 0, true, false, kBf16WgradWaves>), grid, dim3(64 * kBf16WgradWaves),
                         kMainLds, st, (const uint8_t*)a, (const uint8_t*)x, M, N, 2 * ldt, 2 * ldt / splits, nullptr,
                         nullptr, ws, tiles_m, tiles_n, (int)splits, 1, tra, TrOp{});
  }
  if (rc) return rc;
  rc = status();
  if (rc) return rc;
  const int64_t n4 = (int64_t)tiles_m * tiles_n * kTile * kTile / 4;
  if (x_rows)
    hipLaunchKernelGGL((bf16_wgrad_reduce_kernel<true, kBf16WgradWaves>), dim3((unsigned)((n4 + 255) / 256), 1),
                       dim3(256), 0, st, ws, (int)splits, n4, tiles_n, M, N, (uint16_t*)out);
  else
    hipLaunchKernelGGL((bf16_wgrad_reduce_kernel<false, kBf16WgradWaves>), dim3((unsigned)((n4 + 255) / 256), 1),
                       dim3(256), 0, st, ws, (int)splits, n4, tiles_n, M, N, (uint16_t*)out);
  return status();
}

int sfp8_bf16_moe_gemm_wgrad_rows(const void* a, const void* bt, int64_t M, int64_t N, int64_t E, const int* plan,
                                  int64_t ldp, void* out, float* ws, int64_t ws_floats, void* stream) {
  if (!a || !bt || !plan || !out) return kErrNullPointer;
  if (M <= 0 || N <= 0 || E <= 0 || M % 32 || N % 4 || ldp <= 0 || ldp % kTile) return kErrBadShape;
  if (!fits32(slab_rows(M), 2 * ldp) || !fits32(slab_rows(N), 2 * ldp)) return kErrBadShape;
  if (!al16(a) || !al16(bt) || !al16(out) || !al16(ws)) return kErrBadAlignment;
  const int64_t splits = sfp8_moe_wgrad_splits(M, N, E);
  if (!ws || ws_floats < sfp8_bf16_moe_wgrad_workspace_floats(M, N, E)) return kErrWorkspaceTooSmall;
  hipStream_t st = (hipStream_t)stream;
  const int tiles_m = cdiv(M, kTile), tiles_n = cdiv(N, kTile);
  int rc = prep(moe_wgrad_kernel<true, 0, 0, true, false, kBf16WgradWaves>, kMainLds);
  if (rc) return rc;
  hipLaunchKernelGGL((moe_wgrad_kernel<true, 0, 0, true, false, kBf16WgradWaves>),
                     dim3((unsigned)(tiles_m * tiles_n * splits * E)), dim3(64 * kBf16WgradWaves), kMainLds, st,
                     (const uint8_t*)a, (const uint8_t*)bt, M, N, 2 * ldp, nullptr, nullptr, nullptr, ws, plan,
                     tiles_m, tiles_n, (int)splits);
  rc = status();
  if (rc) return rc;
  const int64_t n4 = (int64_t)tiles_m * tiles_n * kTile * kTile / 4;
  hipLaunchKernelGGL((bf16_wgrad_reduce_kernel<false, kBf16WgradWaves>), dim3((unsigned)((n4 + 255) / 256), (unsigned)E),
                     dim3(256), 0, st, ws, (int)splits, n4, tiles_n, M, N, (uint16_t*)out);
  return status();
}

// ---- the weight gradient with row K-slab operands ----
int64_t sfp8_wgrad_rows_workspace_floats(int64_t M, int64_t N, int64_t ldt) {
  return sfp8_wgrad_splits(M, N, ldt) * (int64_t)cdiv(M, kTile) * cdiv(N, kTile) * kTile * kTile;
}

int sfp8_gemm_wgrad_rows(const void* a, int fmt_a, int a_rows, const void* b, int fmt_b, int b_rows, int64_t M,
                         int64_t N, int64_t ldt, const float* sa, const float* sb, float* out, float* ws,
                         int64_t ws_floats, void* stream) {
  if (!sa || !sb || !out || (ldt > 0 && (!a || !b || !ws))) return kErrNullPointer;
  if (M <= 0 || N <= 0 || ldt < 0 || ldt % kTile || N % 4 || !(a_rows || b_rows)) return kErrBadShape;
  if ((a_rows && M % 64) || (b_rows && N % 64)) return kErrBadShape;
  if (fmt_a != kFmtE5M2 || fmt_b != kFmtE4M3) return kErrBadShape;
  if (!fits32(slab_rows(M), ldt) || !fits32(slab_rows(N), ldt)) return kErrBadShape;
  if (!al16(a) || !al16(b) || !al16(out) || !al16(ws)) return kErrBadAlignment;
  hipStream_t st = (hipStream_t)stream;
  if (ldt == 0) {
    const int64_t n = M * N;
    hipLaunchKernelGGL(zero_fill_kernel, dim3((unsigned)((n + 1023) / 1024)), dim3(256), 0, st, out, n);
    return status();
  }
  const int splits = (int)sfp8_wgrad_splits(M, N, ldt);
  if (ws_floats < sfp8_wgrad_rows_workspace_floats(M, N, ldt)) return kErrWorkspaceTooSmall;
  const int rc = wgrad_partials_any(a_rows, b_rows, a, b, M, N, ldt, sa, sb, ws, splits, st);
  if (rc) return rc;
  const int tiles_n = cdiv(N, kTile);
  const int64_t n4 = (int64_t)cdiv(M, kTile) * tiles_n * kTile * kTile / 4;
  if (b_rows)
    hipLaunchKernelGGL((splitk_reduce_kernel<true, kWgradWaves>), dim3((unsigned)((n4 + 255) / 256), 1), dim3(256), 0,
                       st, ws, splits, n4, tiles_n, M, N, sa, sb, out);
  else
    hipLaunchKernelGGL((splitk_reduce_kernel<false, kWgradWaves>), dim3((unsigned)((n4 + 255) / 256), 1), dim3(256), 0,
                       st, ws, splits, n4, tiles_n, M, N, sa, sb, out);
  return status();
}

// ---- the weight gradient fused with the optimizer's momentum stage ----
int64_t sfp8_wgrad_momentum_workspace_floats(int64_t M, int64_t N, int64_t ldt) {
  return sfp8_wgrad_splits(M, N, ldt) * (int64_t)cdiv(M, kTile) * cdiv(N, kTile) * kTile * kTile;
}

int sfp8_gemm_wgrad_momentum(const void* a, int fmt_a, int a_rows, const void* b, int fmt_b, int b_rows, int64_t M,
                             int64_t N, int64_t ldt, const float* sa, const float* sb, float* grad, float* v, void* u,
                             float w_v, float w_u, float* ws, int64_t ws_floats, void* stream) {
  if (!sa || !sb || !v || !u || (ldt > 0 && (!a || !b || !ws))) return kErrNullPointer;
  if (M <= 0 || N <= 0 || ldt < 0 || ldt % kTile || N % 4) return kErrBadShape;
  if ((a_rows && M % 64) || (b_rows && N % 64)) return kErrBadShape;
  if (fmt_a != kFmtE5M2 || fmt_b != kFmtE4M3 || !(w_v > -0.5f && w_v < 0.5f) || !(w_u >= 0.5f)) return kErrBadShape;
  if (!fits32(slab_rows(M), ldt) || !fits32(slab_rows(N), ldt)) return kErrBadShape;
  if (!al16(a) || !al16(b) || !al16(grad) || !al16(v) || !al16(ws) || (((uintptr_t)u) & 7u)) return kErrBadAlignment;
  hipStream_t st = (hipStream_t)stream;
  const int tiles_m = cdiv(M, kTile), tiles_n = cdiv(N, kTile);
  int splits = 0;
  if (ldt > 0) {
    splits = (int)sfp8_wgrad_splits(M, N, ldt);
    if (ws_floats < sfp8_wgrad_momentum_workspace_floats(M, N, ldt)) return kErrWorkspaceTooSmall;
    const int rc = wgrad_partials_any(a_rows, b_rows, a, b, M, N, ldt, sa, sb, ws, splits, st);
    if (rc) return rc;
  }
  const int64_t n4 = (int64_t)tiles_m * tiles_n * kTile * kTile / 4;
  if (b_rows)
    hipLaunchKernelGGL((splitk_momentum_kernel<true, kWgradWaves>), dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st,
                       ws, splits, n4, tiles_n, M, N, sa, sb, grad, v, (uint16_t*)u, w_v, 1.0f - w_u);
  else
    hipLaunchKernelGGL((splitk_momentum_kernel<false, kWgradWaves>), dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st,
                       ws, splits, n4, tiles_n, M, N, sa, sb, grad, v, (uint16_t*)u, w_v, 1.0f - w_u);
  return status();
}

}  // extern "C"
