// Pipelined MFMA main loop for C = A * B^T with K-contiguous A and B rows
// (gfx950).
//
// Tile: 256 A rows x 32*NB*WN B rows, one work-group of (8/TB) x WN waves;
// each wave owns 32*TB A rows x 32*NB B rows as TB x NB MFMA 32x32
// accumulators (fp32, 16*TB*NB registers per lane).  The GEMMs here use
// 8 waves (two per SIMD) of 128 x 64 (TB = 4, NB = 2, WN = 4) per 256 x 256
// tile, or of 64 x 64 (TB = 2, NB = 2, WN = 2) per 256 x 128 tile, so that
// one wave's stage waits and barriers are covered by the other's MFMAs; 4
// waves of 128 x 128 (NB = 4, WN = 2) remain available.
//
// K advances in 64-byte stages through a ring of STAGES LDS buffers, each A
// (16 KiB) + B (64*NB*64 bytes); A stages first, then B stages.
// A 64-byte LDS row r holds its 16-byte chunk c at chunk (c ^ ((r >> 2) & 3)).
// gfx950's LDS serves a 16-byte-per-lane read 16 lanes at a time over 64
// banks (256 bytes); with this swizzle the 16 rows a lane group reads land on
// 16 distinct 4-bank groups.  The DMA fills are contiguous 1 KiB writes.
//
// Global -> LDS: buffer_load_dwordx4 ... lds (one 1 KiB block of 16 rows per
// wave instruction, 4 + NB per wave per stage), issued STAGES-1 stages ahead.
// Row offsets go in the per-lane voffset, the stage offset in soffset.  For
// row-major operands the descriptor's range check returns zeros for rows past
// the operand's end (their voffset alone is out of range), so tail tiles need
// no clamping; K-slab operands are row-padded so every read is in bounds.
//
// Per stage kt (branch-free body):
//   wait until stage kt+1 has landed (vmcnt: younger stages may be in
//   flight), barrier; issue the DMA for stage kt+STAGES-1 into the buffer
//   stage kt-1 used; read the fragments of stage kt+1 into the spare register
//   set; run the MFMAs of stage kt on the current set, interleaved with the
//   reads and the DMA issues.  Stages past the end re-load the last stage into
//   a buffer nobody reads, and read fragments nobody uses.
#pragma once
#include <type_traits>

#include "common.h"

namespace sfp8 {

constexpr int kTile = 256;
constexpr int kStage = 64;                   // bytes of K per stage
constexpr int kStages = 4;                   // LDS ring depth (>= 3)
constexpr int kStageA = kTile * kStage;      // 16 KiB
constexpr int kMainLds = 2 * kStages * kStageA;  // 128 KiB: the 256 x 256 tile's ring

typedef __attribute__((address_space(3))) void* lds_ptr_t;

SFP8_DEV __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int n = bytes > 0x7fffffffLL ? 0x7fffffff : (bytes < 0 ? 0 : (int)bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}

// The same descriptor as four dwords (base[47:0], stride 0, num_records,
// flags), for DMA issued as inline asm.
SFP8_DEV intx4 make_rsrc4(const void* base, int64_t bytes) {
  const int n = bytes > 0x7fffffffLL ? 0x7fffffff : (bytes < 0 ? 0 : (int)bytes);
  const uint64_t a = (uint64_t)(uintptr_t)base;
  return intx4{(int)(uint32_t)a, (int)((uint32_t)(a >> 32) & 0xffffu), n, 0x00020000};
}

// B rows of a wave column: wave (wm, wn) owns A rows 32*TB*wm.. (TB blocks
// of 32) and NB blocks of 32 B rows:
//   plain:  B rows 32*NB*wn + 32*nb
//   paired: gate/up halves of the B tile (rows [0, 16*NB*WN) gate, the rest
//           up); wave wn owns gate blocks 16*NB*wn + 32*nb (nb < NB/2) and
//           the up blocks at the same offsets in the second half.
// WN = wave columns (2: 4 waves, 4: 8 waves).
template <bool PAIRED, int NB, int WN = 2>
struct BLayout {
  static constexpr int kWaveStride = PAIRED ? 16 * NB : 32 * NB;
  static constexpr int off(int nb) {
    return PAIRED ? (nb < NB / 2 ? 32 * nb : 16 * NB * WN + 32 * (nb - NB / 2)) : 32 * nb;
  }
};

// Interleave N_MFMA MFMAs with N_DS LDS reads (spread over all of them) and
// N_VM DMA issues (spread over the first half).
template <int N_MFMA, int N_DS, int N_VM, int I = 0>
SFP8_DEV void sched_interleave() {
  if constexpr (I < N_MFMA) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    constexpr int ds = (N_DS * (I + 1) + N_MFMA - 1) / N_MFMA - (N_DS * I + N_MFMA - 1) / N_MFMA;
    if constexpr (ds > 0) __builtin_amdgcn_sched_group_barrier(0x100, ds, 0);  // DS read
    constexpr int half = N_MFMA / 2;
    constexpr int vm = I < half ? (N_VM * (I + 1) + half - 1) / half - (N_VM * I + half - 1) / half : 0;
    if constexpr (vm > 0) __builtin_amdgcn_sched_group_barrier(0x020, vm, 0);  // VMEM (DMA)
    sched_interleave<N_MFMA, N_DS, N_VM, I + 1>();
  }
}

// The same with up to N_VALU vector-ALU instructions (other work of the wave,
// such as a deferred epilogue) placed after each MFMA.
template <int N_MFMA, int N_VALU, int N_DS, int N_VM, int I = 0>
SFP8_DEV void sched_interleave_valu() {
  if constexpr (I < N_MFMA) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    __builtin_amdgcn_sched_group_barrier(0x002, N_VALU, 0);  // VALU
    constexpr int ds = (N_DS * (I + 1) + N_MFMA - 1) / N_MFMA - (N_DS * I + N_MFMA - 1) / N_MFMA;
    if constexpr (ds > 0) __builtin_amdgcn_sched_group_barrier(0x100, ds, 0);  // DS read
    constexpr int half = N_MFMA / 2;
    constexpr int vm = I < half ? (N_VM * (I + 1) + half - 1) / half - (N_VM * I + half - 1) / half : 0;
    if constexpr (vm > 0) __builtin_amdgcn_sched_group_barrier(0x020, vm, 0);  // VMEM (DMA)
    sched_interleave_valu<N_MFMA, N_VALU, N_DS, N_VM, I + 1>();
  }
}

// TR_A / TR_B: the operand's tile arrives as blocks of 64 (fp8) or 32 (bf16)
// rows, each [tokens of the K stage][64 bytes of 64 (32) M or N values] -- a
// row K-slab (or the row-major rows) of the token-major activation a weight
// gradient reduces over -- and each fragment is assembled from four
// transposing reads (ds_read_b64_tr_b8: 8 tokens of one column per lane;
// ds_read_b64_tr_b16: 4 tokens) in the same (lane half, K) order as the plain
// reads, so the MFMAs see the same values.  Only for a plain (unpaired) B of
// 256 rows.  With TR_B the B tile is not permuted: accumulator v of block nb
// in lane half g is column 32 nb + 8 (v / 4) + 4 g + v % 4 of the wave's
// 32 NB.  These
// instantiations issue their DMA as inline asm: the compiler treats a
// transposing read as possibly aliasing any LDS DMA it knows to be in flight
// and would wait for all of it first; the stage waits and barriers already
// order every read after its stage's DMA.
// TB = A blocks of 32 rows per wave: 4 (two wave rows of 128) or 2 (four
// wave rows of 64; only the fragment, DMA and MFMA pieces, not run()).
template <bool BF16, int FMT_A, int FMT_B, bool PAIRED, int NB = 4, int STAGES = kStages, int PRE = 0,
          bool TR_A = false, bool TR_B = false, int WN = 2, int TB = 4>
struct MainLoop {
  static_assert(TB == 4 || TB == 2, "2 or 4 A blocks per wave");
  static constexpr int kWM = 8 / TB;                        // wave rows
  static constexpr int kWaves = kWM * WN;
  static_assert(!(TR_A || TR_B) || (!PAIRED && 32 * NB * WN == 256), "transposing reads: plain, 256 x 256");
  static constexpr bool kTr = TR_A || TR_B;
  using Rsrc = typename std::conditional<kTr, intx4, __amdgpu_buffer_rsrc_t>::type;
  static SFP8_DEV Rsrc rsrc(const void* base, int64_t bytes) {
    if constexpr (kTr) return make_rsrc4(base, bytes);
    else return make_rsrc(base, bytes);
  }
  // One 16-byte-per-lane DMA into LDS at dst (wave-uniform)
  static SFP8_DEV void dma16(uint8_t* dst, Rsrc r, uint32_t voff, int soff) {
    if constexpr (kTr) {
      const uint32_t m0v = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_ptr_t)dst);
      asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                   :: "s"(m0v), "v"(voff), "s"(r), "s"(soff) : "memory");
    } else {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)dst, 16, voff, soff, 0, 0);
    }
  }
  static_assert(NB == 2 || NB == 4, "2 or 4 B blocks per wave");
  static_assert(STAGES >= 3, "at least three LDS stages");
  static constexpr int kTileN = 32 * NB * WN;             // B rows per tile
  static constexpr int kStageB = kTileN * kStage;
  static constexpr int kLdsB = STAGES * kStageA;           // start of the B stages
  static constexpr int kLds = STAGES * (kStageA + kStageB);
  static constexpr int kDmaA = 16 / kWaves;                // A DMA instructions per wave per stage
  static constexpr int kDmaB = kTileN / 16 / kWaves;
  static constexpr int kDma = kDmaA + kDmaB;               // DMA instructions per wave per stage
  using Acc = floatx16[TB][NB];

  // DMA instruction j of this wave's share of one stage: J < 4 are A blocks,
  // the rest B blocks (16 rows = 1 KiB each).
  static SFP8_DEV void load_one(int j, uint8_t* lds, int buf, Rsrc ra,
                                Rsrc rb, const uint32_t (&voff_a)[4], const uint32_t (&voff_b)[NB],
                                int soff_a, int soff_b, int wave) {
    if (j < kDmaA) {
      uint8_t* dst = lds + buf * kStageA + ((kTile / kWaves) * wave + 16 * j) * kStage;
      dma16(dst, ra, voff_a[j], soff_a);
    } else {
      uint8_t* dst = lds + kLdsB + buf * kStageB + ((kTileN / kWaves) * wave + 16 * (j - kDmaA)) * kStage;
      dma16(dst, rb, voff_b[j - kDmaA], soff_b);
    }
  }

  // Issue this wave's DMA instructions of one stage.
  static SFP8_DEV void load_stage(uint8_t* lds, int buf, Rsrc ra, Rsrc rb,
                                  const uint32_t (&voff_a)[4], const uint32_t (&voff_b)[NB], int soff_a, int soff_b,
                                  int wave) {
#pragma unroll
    for (int j = 0; j < kDma; ++j) load_one(j, lds, buf, ra, rb, voff_a, voff_b, soff_a, soff_b, wave);
  }

  // Fragments of one stage: per block 32 bytes per lane (lane half g holds
  // logical chunks 2g, 2g+1 in the low / high 16 bytes).
  struct Frag {
    intx8 a[TB];
    intx8 b[NB];
  };

  // Fragment I of one stage (I < TB: A block I, else B block I - TB): two
  // 16-byte LDS reads.
  // Four transposing reads of one block of a TR operand tile: block k (32
  // columns) lives in 64-column slab k / 2; off[2 q + (k & 1)] addresses
  // read q (K bytes 8 q .. 8 q + 7 of the lane half's 32).
  template <int K>
  static SFP8_DEV intx8 read_tr_block(const uint8_t* p, const uint32_t (&off)[8]) {
    if constexpr (BF16) {
      // bf16: block k is 32-row slab k; read q returns tokens 4 q .. 4 q + 3
      // of the lane half's 16 (the two MFMA steps' 8 each)
      const uint8_t* q = p + K * (32 * kStage);
      const intx2 r0 = lds_read_tr16(q + off[0]);
      const intx2 r1 = lds_read_tr16(q + off[1]);
      const intx2 r2 = lds_read_tr16(q + off[2]);
      const intx2 r3 = lds_read_tr16(q + off[3]);
      return intx8{r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
    } else {
      const uint8_t* q = p + (K >> 1) * (64 * kStage);
      const intx2 r0 = lds_read_tr8(q + off[0 + (K & 1)]);
      const intx2 r1 = lds_read_tr8(q + off[2 + (K & 1)]);
      const intx2 r2 = lds_read_tr8(q + off[4 + (K & 1)]);
      const intx2 r3 = lds_read_tr8(q + off[6 + (K & 1)]);
      return intx8{r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
    }
  }

  template <int I>
  static SFP8_DEV void read_frag(const uint8_t* lds, int buf, const uint32_t (&aoff)[8], const uint32_t (&boff)[8],
                                 Frag& f) {
    if constexpr (I < TB) {
      if constexpr (TR_A) {
        f.a[I] = read_tr_block<I>(lds + buf * kStageA, aoff);
      } else {
        const uint8_t* p = lds + buf * kStageA + I * 32 * kStage;
        const intx4 lo = *reinterpret_cast<const intx4*>(p + aoff[0]);
        const intx4 hi = *reinterpret_cast<const intx4*>(p + aoff[1]);
        f.a[I] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
    } else {
      if constexpr (TR_B) {
        f.b[I - TB] = read_tr_block<I - TB>(lds + kLdsB + buf * kStageB, boff);
      } else {
        const uint8_t* p = lds + buf * kStageB + BLayout<PAIRED, NB, WN>::off(I - TB) * kStage;
        const intx4 lo = *reinterpret_cast<const intx4*>(p + boff[0]);
        const intx4 hi = *reinterpret_cast<const intx4*>(p + boff[1]);
        f.b[I - TB] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
    }
  }

  template <int I = 0>
  static SFP8_DEV void read_frags(const uint8_t* lds, int buf, const uint32_t (&aoff)[8], const uint32_t (&boff)[8],
                                  Frag& f) {
    if constexpr (I < TB + NB) {
      read_frag<I>(lds, buf, aoff, boff, f);
      read_frags<I + 1>(lds, buf, aoff, boff, f);
    }
  }

  static constexpr int kMfma = (BF16 ? 2 : 1) * TB * NB;  // MFMAs per stage
  // MFMAs of a stage issued before its barrier: they need only registers, and
  // keep the matrix pipe busy while the waves meet.
  static constexpr int kPre = PRE;

  // MFMAs [LO, HI) of one stage, in (h, tb, nb) order.
  template <int LO, int HI>
  static SFP8_DEV void mfma_range(const Frag& f, Acc& acc) {
#pragma unroll
    for (int i = LO; i < HI; ++i) {
      if constexpr (!BF16) {
        const int tb = i / NB, nb = i % NB;
        // B fragment first: each lane's accumulator is one A row (m)
        acc[tb][nb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.b[nb], f.a[tb], acc[tb][nb], FMT_B, FMT_A,
                                                                      0, 0, 0, 0);
      } else {
        const int h = i / (TB * NB), tb = (i / NB) % TB, nb = i % NB;
        const bf16x8 av = __builtin_bit_cast(
            bf16x8, h ? __builtin_shufflevector(f.a[tb], f.a[tb], 4, 5, 6, 7)
                      : __builtin_shufflevector(f.a[tb], f.a[tb], 0, 1, 2, 3));
        const bf16x8 bv = __builtin_bit_cast(
            bf16x8, h ? __builtin_shufflevector(f.b[nb], f.b[nb], 4, 5, 6, 7)
                      : __builtin_shufflevector(f.b[nb], f.b[nb], 0, 1, 2, 3));
        acc[tb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bv, av, acc[tb][nb], 0, 0, 0);
      }
    }
  }

  // Per stage after the barrier: kMfma - kPre MFMAs, 2*(4+NB) LDS reads, 4+NB DMAs.
  static SFP8_DEV void schedule() { sched_interleave<kMfma - kPre, 2 * (4 + NB), kDma>(); }

  // MFMA M of the stage, then fragment reads [R0, R1) of the next stage, as
  // one group the scheduler may not reorder with its neighbours.
  template <int M, int R0, int R1>
  static SFP8_DEV void mfma_then_reads(const uint8_t* lds, const Frag& cur, Frag& nxt, Acc& acc, int rd_buf,
                                       const uint32_t (&aoff)[8], const uint32_t (&boff)[8]) {
    mfma_range<M, M + 1>(cur, acc);
    if constexpr (R0 < R1) read_frag<R0>(lds, rd_buf, aoff, boff, nxt);
    if constexpr (R0 + 1 < R1) read_frag<R0 + 1>(lds, rd_buf, aoff, boff, nxt);
    __builtin_amdgcn_sched_barrier(0);
  }

  // MFMA M of the stage, then DMA instructions [J0, J1) of stage `ld`.
  template <int M, int J0, int J1>
  static SFP8_DEV void mfma_then_dma(uint8_t* lds, const Frag& cur, Acc& acc, int dma_buf,
                                     Rsrc ra, Rsrc rb,
                                     const uint32_t (&voff_a)[4], const uint32_t (&voff_b)[NB], int soff_a,
                                     int soff_b, int wave) {
    mfma_range<M, M + 1>(cur, acc);
    if constexpr (J0 < J1) load_one(J0, lds, dma_buf, ra, rb, voff_a, voff_b, soff_a, soff_b, wave);
    if constexpr (J0 + 1 < J1) load_one(J0 + 1, lds, dma_buf, ra, rb, voff_a, voff_b, soff_a, soff_b, wave);
    __builtin_amdgcn_sched_barrier(0);
  }

  // One stage, in a fixed order:
  //   kSchedPre MFMAs of stage kt (registers only: they keep the matrix pipe busy
  //   while the waves meet at the barrier);
  //   wait for stage kt+1 to land, barrier;
  //   MFMAs, each followed by a group of the 4+NB fragments (two 16-byte
  //   reads each) of stage kt+1 from `rd_buf` or of the 4+NB DMA
  //   instructions of stage `ld` into `dma_buf` (the buffer stage kt-1 used:
  //   every wave finished reading it before this barrier), all within the
  //   first 10-16 MFMAs so the reads land long before stage kt+1 starts;
  //   the remaining MFMAs.
  // The grouping depends on the MFMA length: fp8 256 x 256 alternates
  // fragments and DMA over 10 MFMAs of 64 cycles, bf16 alternates one
  // fragment and one DMA over 16 MFMAs of 32 cycles, NB = 2 issues the
  // fragments over 3 MFMAs and then the DMA over 3.
  static constexpr int kSchedPre = 2;
  static_assert(TB != 4 || kMfma >= kSchedPre + (4 + NB) / 2 + (4 + NB) / 2, "stage too short for the schedule");
  static SFP8_DEV void stage(uint8_t* lds, const Frag& cur, Frag& nxt, Acc& acc, int dma_buf, int ld, int rd_buf,
                             Rsrc ra, Rsrc rb, const uint32_t (&voff_a)[4],
                             const uint32_t (&voff_b)[NB], int a_sstride, int b_sstride, const uint32_t (&aoff)[8],
                             const uint32_t (&boff)[8], int wave) {
    constexpr int P = kSchedPre;
    mfma_range<0, P>(cur, acc);
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kDma * (STAGES - 3)) : "memory");
    __builtin_amdgcn_sched_barrier(0);
    const int sa = ld * a_sstride, sb = ld * b_sstride;
    constexpr int H = (4 + NB) / 2;  // MFMAs carrying reads (and DMA issues)
    if constexpr (BF16 && NB == 4) {
      // bf16: 32 MFMAs of 32 cycles per stage.  Two reads after each of 4
      // MFMAs would crowd 16 KiB of LDS reads per wave into 128 cycles; one
      // fragment and one DMA instruction after alternate MFMAs spread them
      // over 16 (5 % faster on the down dgrad than the fp8 order).
      mfma_then_reads<P + 0, 0, 1>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_dma<P + 1, 0, 1>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
      mfma_then_reads<P + 2, 1, 2>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_dma<P + 3, 1, 2>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
      mfma_then_reads<P + 4, 2, 3>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_dma<P + 5, 2, 3>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
      mfma_then_reads<P + 6, 3, 4>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_dma<P + 7, 3, 4>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
      mfma_then_reads<P + 8, 4, 5>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_dma<P + 9, 4, 5>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
      mfma_then_reads<P + 10, 5, 6>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_dma<P + 11, 5, 6>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
      mfma_then_reads<P + 12, 6, 7>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_dma<P + 13, 6, 7>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
      mfma_then_reads<P + 14, 7, 8>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_dma<P + 15, 7, 8>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
      mfma_range<P + 16, kMfma>(cur, acc);
      __builtin_amdgcn_sched_barrier(0);
      return;
    }
    if constexpr (BF16 && NB == 2) {
      // bf16, 8 waves of 128 x 64: 16 MFMAs of 32 cycles; six fragments and
      // four DMA issues alternate over 10 of them
      mfma_then_reads<P + 0, 0, 1>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_dma<P + 1, 0, 1>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
      mfma_then_reads<P + 2, 1, 2>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_dma<P + 3, 1, 2>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
      mfma_then_reads<P + 4, 2, 3>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_dma<P + 5, 2, 3>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
      mfma_then_reads<P + 6, 3, 4>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_dma<P + 7, 3, 4>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
      mfma_then_reads<P + 8, 4, 5>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_reads<P + 9, 5, 6>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_range<P + 10, kMfma>(cur, acc);
      __builtin_amdgcn_sched_barrier(0);
      return;
    }
    if constexpr (!BF16 && NB == 4) {
      // fp8, 256 x 256: fragments and DMA issues alternate over 10 MFMAs
      // (2-3 % faster than 4 MFMAs of reads followed by 4 of DMA)
      mfma_then_reads<P + 0, 0, 1>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_dma<P + 1, 0, 1>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
      mfma_then_reads<P + 2, 1, 3>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_dma<P + 3, 1, 3>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
      mfma_then_reads<P + 4, 3, 5>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_dma<P + 5, 3, 5>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
      mfma_then_reads<P + 6, 5, 7>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_dma<P + 7, 5, 7>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
      mfma_then_reads<P + 8, 7, 8>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_dma<P + 9, 7, 8>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
      mfma_range<P + 10, kMfma>(cur, acc);
      __builtin_amdgcn_sched_barrier(0);
      return;
    }
    if constexpr (!BF16 && NB == 2 && kDma == 4 && TR_A && TR_B) {
      // fp8, 8 waves of 128 x 64, both operands through transposing reads
      // (four per fragment): two fragments and two DMA issues alternate over
      // 5 MFMAs (2 % faster on the gate/up weight gradient than the order
      // below, which the plain reads prefer)
      mfma_then_reads<P + 0, 0, 2>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_dma<P + 1, 0, 2>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
      mfma_then_reads<P + 2, 2, 4>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_dma<P + 3, 2, 4>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
      mfma_then_reads<P + 4, 4, 6>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_range<P + 5, kMfma>(cur, acc);
      __builtin_amdgcn_sched_barrier(0);
      return;
    }
    if constexpr (!BF16 && NB == 2 && kDma == 4) {
      // fp8, 8 waves of 128 x 64: 8 MFMAs of 64 cycles; two fragments after
      // each of 3, then two DMA issues after each of 2
      mfma_then_reads<P + 0, 0, 2>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_reads<P + 1, 2, 4>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_reads<P + 2, 4, 6>(lds, cur, nxt, acc, rd_buf, aoff, boff);
      mfma_then_dma<P + 3, 0, 2>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
      mfma_then_dma<P + 4, 2, 4>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
      mfma_range<P + 5, kMfma>(cur, acc);
      __builtin_amdgcn_sched_barrier(0);
      return;
    }
    // NB = 2: two fragments after each of 3 MFMAs, then two DMA issues after
    // each of 3
    mfma_then_reads<P + 0, 0, 2>(lds, cur, nxt, acc, rd_buf, aoff, boff);
    mfma_then_reads<P + 1, 2, 4>(lds, cur, nxt, acc, rd_buf, aoff, boff);
    mfma_then_reads<P + 2, 4, 6>(lds, cur, nxt, acc, rd_buf, aoff, boff);
    mfma_then_dma<P + H + 0, 0, 2>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
    mfma_then_dma<P + H + 1, 2, 4>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
    mfma_then_dma<P + H + 2, 4, 6>(lds, cur, acc, dma_buf, ra, rb, voff_a, voff_b, sa, sb, wave);
    mfma_range<P + 2 * H, kMfma>(cur, acc);
    __builtin_amdgcn_sched_barrier(0);
  }

  // a_bytes/b_bytes: bytes available from a_base/b_base (range-checked);
  // a_rowoff(r)/b_rowoff(r): byte offset of tile row r from the base within
  // one K stage; a_sstride/b_sstride: bytes from one 64-byte K stage to the
  // next (64 for row-major operands, rows * 64 for K-slab operands);
  // nk: number of K stages, even.
  template <class ARow, class BRow>
  static SFP8_DEV void run(uint8_t* lds, const uint8_t* a_base, int64_t a_bytes, ARow a_rowoff, int a_sstride,
                           const uint8_t* b_base, int64_t b_bytes, BRow b_rowoff, int b_sstride, int nk, Acc& acc) {
    static_assert(TB == 4, "run() schedules four A blocks per wave");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const Rsrc ra = rsrc(a_base, a_bytes);
    const Rsrc rb = rsrc(b_base, b_bytes);
    // DMA lane offsets: A instruction j covers tile rows 64*wave + 16*j + lane/4,
    // B instruction j rows 16*NB*wave + 16*j + lane/4; physical chunk lane%4
    // <- logical chunk (lane%4) ^ ((row >> 2) & 3)
    uint32_t voff_a[4], voff_b[NB];
    const uint32_t chunk = (uint32_t)(((lane & 3) ^ ((lane >> 4) & 3)) << 4);
    // fp8 TR operands: chunk c of row r at c ^ (2 * ((r >> 2) & 1)), so that
    // the 8 rows x 2 chunks a half-wave's transposing read touches fill the
    // 64 banks (rows r and r + 4 share banks under the plain swizzle).  bf16
    // TR operands: unswizzled (a half-wave reads 4 whole 64-byte rows).
    const uint32_t chunk_tr =
        BF16 ? (uint32_t)((lane & 3) << 4) : (uint32_t)(((lane & 3) ^ (((lane >> 4) & 1) << 1)) << 4);
#pragma unroll
    for (int j = 0; j < kDmaA; ++j)
      voff_a[j] = (uint32_t)a_rowoff((kTile / kWaves) * wave + 16 * j + (lane >> 2)) + (TR_A ? chunk_tr : chunk);
#pragma unroll
    for (int j = 0; j < kDmaB; ++j)
      voff_b[j] = (uint32_t)b_rowoff((kTileN / kWaves) * wave + 16 * j + (lane >> 2)) + (TR_B ? chunk_tr : chunk);
    // fragment read offsets (lane half g reads logical chunks 2g, 2g+1)
    const int fr = lane & 31, g = lane >> 5;
    const int sw = (fr >> 2) & 3;
    uint32_t aoff[8], boff[8];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      aoff[h] = (uint32_t)((128 * wm + fr) * kStage + (((2 * g + h) ^ sw) << 4));
      boff[h] = (uint32_t)(kLdsB + (BLayout<PAIRED, NB, WN>::kWaveStride * wn + fr) * kStage + (((2 * g + h) ^ sw) << 4));
    }
    if constexpr (kTr && BF16) {
      // bf16 transposing reads: 16-lane group G = lane / 16 (lane half G / 2,
      // column half G % 2 of the slab's 32 columns); for read q lane 16 G + j
      // addresses token 16 (G / 2) + 4 q + j / 4 and columns 16 (G % 2) +
      // 4 (j % 4) .. + 3; the read returns to lane 16 G + 4 a + b tokens
      // 16 (G / 2) + 4 q .. + 3 of column 16 (G % 2) + 4 a + b.  Slabs of the
      // wave's rows: 4 wm (A) or NB wn (B).
      const int G = lane >> 4, j = lane & 15;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int tok = 16 * (G >> 1) + 4 * q + (j >> 2);
        const uint32_t cb = (uint32_t)(32 * (G & 1) + 8 * (j & 3));
        if constexpr (TR_A) aoff[q] = (uint32_t)((128 * wm + tok) * kStage) + cb;
        if constexpr (TR_B) boff[q] = (uint32_t)((32 * NB * wn + tok) * kStage) + cb;
      }
    } else if constexpr (kTr) {
      // Transposing reads: 16-lane group G = lane / 16 (lane half g = G / 2,
      // column half G % 2 of the block's 32 columns); within it lane 2b + h
      // addresses tile row (token) 32 g + 8 q + b of the block's slab and the
      // 8 bytes 8 h.. of logical chunk 2 (k & 1) + G % 2 (at its TR swizzle
      // position); the read returns to lane i rows 32 g + 8 q .. + 7 of column
      // 16 (G % 2) + i.  Slab of the wave's rows: 2 wm (A) or NB wn / 2 (B).
      const int G = lane >> 4, li = lane & 15, bq = li >> 1, hb = li & 1, gh = G >> 1, gc = G & 1;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int k1 = 0; k1 < 2; ++k1) {
          const int rr = 32 * gh + 8 * q + bq;  // row within the 64-row slab
          const uint32_t cb = (uint32_t)((((2 * k1 + gc) ^ (((rr >> 2) & 1) << 1)) << 4) + 8 * hb);
          if constexpr (TR_A) aoff[2 * q + k1] = (uint32_t)((128 * wm + rr) * kStage) + cb;
          if constexpr (TR_B) boff[2 * q + k1] = (uint32_t)((32 * NB * wn + rr) * kStage) + cb;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j) acc[i][j] = floatx16{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f,
                                                        0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const int last = nk - 1;
    // Stages past the last keep their DMA instructions (the waits count
    // them) but read through descriptors of zero records: every lane is out
    // of range, so no memory is read and the unused ring slot gets zeros.
    const Rsrc ra0 = rsrc(a_base, 0);
    const Rsrc rb0 = rsrc(b_base, 0);
    // prologue: stages 0 .. STAGES-2 in flight; stage 0 landed; its fragments read
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s) {
      const bool live = s <= last;
      const int ld = live ? s : last;
      load_stage(lds, s, live ? ra : ra0, live ? rb : rb0, voff_a, voff_b, ld * a_sstride, ld * b_sstride, wave);
    }
    // kDma DMA instructions per wave per stage: stages 1 .. STAGES-2 may still fly
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kDma * (STAGES - 2)) : "memory");
    Frag f0, f1;
    read_frags(lds, 0, aoff, boff, f0);
    // two stages per trip so the register sets alternate statically (nk is even).
    // Stage s lives in ring buffer s % STAGES; at stage kt the DMA refills the
    // buffer of stage kt-1, whose fragments were consumed one stage earlier.
    for (int kt = 0; kt < nk; kt += 2) {
      // stage kt on f0, prefetch stage kt+1 into f1; stages kt+2 .. kt+STAGES-2 may fly
      {
        const bool live = kt + STAGES - 1 <= last;
        const int ld = live ? kt + STAGES - 1 : last;
        stage(lds, f0, f1, acc, (kt + STAGES - 1) % STAGES, ld, (kt + 1) % STAGES, live ? ra : ra0,
              live ? rb : rb0, voff_a, voff_b, a_sstride, b_sstride, aoff, boff, wave);
      }
      // stage kt+1 on f1, prefetch stage kt+2 into f0
      {
        const bool live = kt + STAGES <= last;
        const int ld = live ? kt + STAGES : last;
        stage(lds, f1, f0, acc, kt % STAGES, ld, (kt + 2) % STAGES, live ? ra : ra0, live ? rb : rb0, voff_a,
              voff_b, a_sstride, b_sstride, aoff, boff, wave);
      }
    }
    // drain the (empty) DMA still in flight before the LDS is reused
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  }
};

}  // namespace sfp8
