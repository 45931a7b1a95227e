// Pipelined MFMA main loop for C = A * B^T with K-contiguous A and B rows
// (gfx950, one 256-thread work-group = 4 waves, one wave per SIMD).
//
// Tile: 256 A rows x 256 B rows; each wave owns a 128 x 128 block grid of
// 4 x 4 MFMA 32x32 accumulators (fp32, 256 registers per lane).
//
// K advances in 64-byte stages.  Four LDS stages of (A 16 KiB + B 16 KiB):
//   A stage s at s*16 KiB, B stage s at 64 KiB + s*16 KiB.
// A 64-byte LDS row r holds its 16-byte chunk c at chunk (c ^ ((r >> 2) & 3)).
// gfx950's LDS serves a 16-byte-per-lane read 16 lanes at a time over 64
// banks (256 bytes); with this swizzle the 16 rows a lane group reads land on
// 16 distinct 4-bank groups.  The DMA fills are contiguous 1 KiB writes.
//
// Global -> LDS: buffer_load_dwordx4 ... lds (one 1 KiB block of 16 rows per
// wave instruction, 8 per wave per stage), issued three stages ahead.  Row
// offsets go in the per-lane voffset, the stage offset in soffset.  For
// row-major operands the descriptor's range check returns zeros for rows past
// the operand's end (their voffset alone is out of range), so tail tiles need
// no clamping; K-slab operands are row-padded so every read is in bounds.
//
// Per stage kt (branch-free body):
//   wait until stage kt+1 has landed (vmcnt: one younger stage may be in
//   flight), barrier; issue the DMA for stage kt+3 into the buffer stage kt-1
//   used; read the fragments of stage kt+1 into the spare register set; run
//   the MFMAs of stage kt on the current set, interleaved with the reads and
//   the DMA issues.  Stages past the end re-load the last stage into a buffer
//   nobody reads, and read fragments nobody uses.
#pragma once
#include "common.h"

namespace sfp8 {

constexpr int kTile = 256;
constexpr int kStage = 64;                   // bytes of K per stage
constexpr int kStages = 4;                   // LDS ring depth (>= 3)
constexpr int kStageA = kTile * kStage;      // 16 KiB
constexpr int kLdsB = kStages * kStageA;     // 64 KiB: start of the B stages
constexpr int kMainLds = 2 * kStages * kStageA;  // 128 KiB
constexpr int kFmtE4M3 = 0;
constexpr int kFmtE5M2 = 1;

typedef __attribute__((address_space(3))) void* lds_ptr_t;

SFP8_DEV __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int n = bytes > 0x7fffffffLL ? 0x7fffffff : (bytes < 0 ? 0 : (int)bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}

// Wave-level B block layout inside the 256-row B tile.
//   plain:  wave column wn owns B rows 128*wn + {0, 32, 64, 96}
//   paired: wave column wn owns B rows 64*wn + {0, 32, 128, 160}  (gate/up pairs)
template <bool PAIRED>
struct BLayout {
  static constexpr int kWaveStride = PAIRED ? 64 : 128;
  static constexpr int kOff[4] = {0, 32, PAIRED ? 128 : 64, PAIRED ? 160 : 96};
};

template <bool BF16, int FMT_A, int FMT_B, bool PAIRED>
struct MainLoop {
  // Issue this wave's 8 DMA instructions of one stage.
  static SFP8_DEV void load_stage(uint8_t* lds, int buf, __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb,
                                  const uint32_t (&voff_a)[4], const uint32_t (&voff_b)[4], int soff_a, int soff_b,
                                  int wave) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint8_t* dst = lds + buf * kStageA + (64 * wave + 16 * j) * kStage;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)dst, 16, voff_a[j], soff_a, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint8_t* dst = lds + kLdsB + buf * kStageA + (64 * wave + 16 * j) * kStage;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)dst, 16, voff_b[j], soff_b, 0, 0);
    }
  }

  // Fragments of one stage: per block 32 bytes per lane (lane half g holds
  // logical chunks 2g, 2g+1 in the low / high 16 bytes).
  struct Frag {
    intx8 a[4];
    intx8 b[4];
  };

  static SFP8_DEV void read_frags(const uint8_t* lds, int buf, const uint32_t (&aoff)[2], const uint32_t (&boff)[2],
                                  Frag& f) {
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      const uint8_t* p = lds + buf * kStageA + tb * 32 * kStage;
      const intx4 lo = *reinterpret_cast<const intx4*>(p + aoff[0]);
      const intx4 hi = *reinterpret_cast<const intx4*>(p + aoff[1]);
      f.a[tb] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const uint8_t* p = lds + buf * kStageA + BLayout<PAIRED>::kOff[nb] * kStage;
      const intx4 lo = *reinterpret_cast<const intx4*>(p + boff[0]);
      const intx4 hi = *reinterpret_cast<const intx4*>(p + boff[1]);
      f.b[nb] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
  }

  static SFP8_DEV void mfma_stage(const Frag& f, floatx16 (&acc)[4][4]) {
    if constexpr (!BF16) {
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
          // B fragment first: each lane's accumulator is one A row (m)
          acc[tb][nb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.b[nb], f.a[tb], acc[tb][nb], FMT_B, FMT_A,
                                                                        0, 0, 0, 0);
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb)
#pragma unroll
          for (int nb = 0; nb < 4; ++nb) {
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

  // Interleave: MFMA, LDS read, DMA issue -- per stage 16 (fp8) or 32 (bf16)
  // MFMAs, 16 LDS reads, 8 DMAs.
  static SFP8_DEV void schedule() {
    constexpr int kMfma = BF16 ? 32 : 16;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM (DMA)
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, kMfma - 16, 0);
  }

  // a_bytes/b_bytes: bytes available from a_base/b_base (range-checked);
  // a_rowoff(r)/b_rowoff(r): byte offset of tile row r (0..255) from the base
  // within one K stage; a_sstride/b_sstride: bytes from one 64-byte K stage to
  // the next (64 for row-major operands, rows * 64 for K-slab operands);
  // nk: number of K stages, even.
  template <class ARow, class BRow>
  static SFP8_DEV void run(uint8_t* lds, const uint8_t* a_base, int64_t a_bytes, ARow a_rowoff, int a_sstride,
                           const uint8_t* b_base, int64_t b_bytes, BRow b_rowoff, int b_sstride, int nk,
                           floatx16 (&acc)[4][4]) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(a_base, a_bytes);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(b_base, b_bytes);
    // DMA lane offsets: instruction j covers tile rows 64*wave + 16*j + lane/4,
    // physical chunk lane%4 <- logical chunk (lane%4) ^ ((row >> 2) & 3)
    uint32_t voff_a[4], voff_b[4];
    const uint32_t chunk = (uint32_t)(((lane & 3) ^ ((lane >> 4) & 3)) << 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = 64 * wave + 16 * j + (lane >> 2);
      voff_a[j] = (uint32_t)a_rowoff(r) + chunk;
      voff_b[j] = (uint32_t)b_rowoff(r) + chunk;
    }
    // fragment read offsets (lane half g reads logical chunks 2g, 2g+1)
    const int fr = lane & 31, g = lane >> 5;
    const int sw = (fr >> 2) & 3;
    uint32_t aoff[2], boff[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      aoff[h] = (uint32_t)((128 * wm + fr) * kStage + (((2 * g + h) ^ sw) << 4));
      boff[h] = (uint32_t)(kLdsB + (BLayout<PAIRED>::kWaveStride * wn + fr) * kStage + (((2 * g + h) ^ sw) << 4));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = floatx16{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f,
                                                       0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const int last = nk - 1;
    // prologue: stages 0 .. kStages-2 in flight; stage 0 landed; its fragments read
#pragma unroll
    for (int s = 0; s < kStages - 1; ++s) {
      const int ld = s < last ? s : last;
      load_stage(lds, s, ra, rb, voff_a, voff_b, ld * a_sstride, ld * b_sstride, wave);
    }
    // 8 DMA instructions per wave per stage: stages 1 .. kStages-2 may still fly
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(8 * (kStages - 2)) : "memory");
    Frag f0, f1;
    read_frags(lds, 0, aoff, boff, f0);
    // two stages per trip so the register sets alternate statically (nk is even).
    // Stage s lives in ring buffer s % kStages; at stage kt the DMA refills the
    // buffer of stage kt-1, whose fragments were consumed one stage earlier.
    for (int kt = 0; kt < nk; kt += 2) {
      // stage kt on f0, prefetch stage kt+1 into f1; stages kt+2 .. kt+kStages-2 may fly
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(8 * (kStages - 3)) : "memory");
      {
        const int ld = kt + kStages - 1 < last ? kt + kStages - 1 : last;
        load_stage(lds, (kt + kStages - 1) % kStages, ra, rb, voff_a, voff_b, ld * a_sstride, ld * b_sstride,
                   wave);
        read_frags(lds, (kt + 1) % kStages, aoff, boff, f1);
        mfma_stage(f0, acc);
        schedule();
      }
      // stage kt+1 on f1, prefetch stage kt+2 into f0
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(8 * (kStages - 3)) : "memory");
      {
        const int ld = kt + kStages < last ? kt + kStages : last;
        load_stage(lds, kt % kStages, ra, rb, voff_a, voff_b, ld * a_sstride, ld * b_sstride, wave);
        read_frags(lds, (kt + 2) % kStages, aoff, boff, f0);
        mfma_stage(f1, acc);
        schedule();
      }
    }
    // drain the DMA still in flight before the LDS is reused
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  }
};

}  // namespace sfp8
