// stream.h -- per-wave LDS ring streaming of quantised weight rows (gfx950).
//
// Each wave streams its own contiguous stretch of weight rows HBM -> LDS
// with global_load_lds_dwordx4 (64 lanes x 16 B = 1 KB per instruction,
// lane-linear in LDS, no staging registers) through a ring of S stages, and
// computes on stage i while stages i+1 .. i+S-1 are in flight.
//
// A "step" covers up to kSB consecutive super-blocks of each of NSEG row
// segments (R rows x M matrices).  Stage layout in LDS: segment j occupies
// bytes [j*kSB*B, (j+1)*kSB*B) of the stage, block s of it at j*kSB*B + s*B.
// Chunk c (16 B) of the stage goes to LDS offset 16c; chunks past the valid
// part of a segment (short last step of a row) re-load the segment's first
// chunk into their own (unused) LDS location, so every instruction has all
// lanes active and the per-stage instruction count NI is a compile-time
// constant -- which is what the manual wait below needs.
//
// The compiler does not track the dependence of LDS reads on these DMA
// loads, so the consumer waits explicitly (wait_vmcnt) and the asm carries a
// memory clobber so no LDS read is hoisted above it.
#pragma once

#include "qk_common.h"

namespace rf {

constexpr int kSB = 16;  // super-blocks per segment per step

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt[3:0] | expcnt 7 << 4 |
// lgkmcnt 15 << 8 | vmcnt[5:4] << 14).  Issued through the builtin so the
// compiler's own wait tracking sees it (it then knows the DMA it waited for
// is complete); the empty asm keeps memory accesses from moving across it.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
    asm volatile("" ::: "memory");
}

// Workgroup barrier that does not wait for outstanding memory loads
// (__syncthreads() implies a fence, i.e. vmcnt(0), which would drain the
// weight DMA ring).  LDS writes of this wave are completed first.  DMA data
// must be waited for with wait_vmcnt by the wave that issued it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ void dma16(const void* src, uint8_t* lds_base) {
    __builtin_amdgcn_global_load_lds(src, (lds_ptr_t)lds_base, 16, 0, 0);
}

// Ring reads.  The compiler cannot tell a read of one ring slot from the DMA
// still filling another and would wait for all outstanding DMA before it, so
// ring slots are read with inline-asm ds_reads, invisible to its wait
// tracking.  Each group of reads and its s_waitcnt lgkmcnt(0) form ONE asm
// statement with early-clobber outputs: the compiler treats asm outputs as
// ready when the statement ends, so a wait in a separate statement would let
// it copy a register before the load had written it.  (Its own LDS waits
// only ever count fewer outstanding operations than exist: they may
// over-wait, never under-wait.)
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(lds_ptr_t)(const_cast<void*>(p));
}

// Two Q4_K units: header + the 32 nibble bytes of pair p, from two blocks.
__device__ __forceinline__ void ring_read_q4x2(const uint8_t* b0, const uint8_t* b1, int p, u32x4 (&o)[6]) {
    const uint32_t a0 = lds_addr(b0), a1 = lds_addr(b1), q = 16u + 32u * (uint32_t)p;
    asm volatile(
        "ds_read_b128 %0, %6\n\t"
        "ds_read_b128 %1, %7\n\t"
        "ds_read_b128 %2, %7 offset:16\n\t"
        "ds_read_b128 %3, %8\n\t"
        "ds_read_b128 %4, %9\n\t"
        "ds_read_b128 %5, %9 offset:16\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3]), "=&v"(o[4]), "=&v"(o[5])
        : "v"(a0), "v"(a0 + q), "v"(a1), "v"(a1 + q)
        : "memory");
}

// One Q6_K lane unit: ql-low, ql-high, qh (16 B each), 8 scale bytes and the
// dword holding d (bytes 206..209).
__device__ __forceinline__ void ring_read_q6(const uint8_t* blk, int p, u32x4& lo, u32x4& hi, u32x4& qh, u32x2& sc,
                                             uint32_t& d) {
    const int n = p >> 1, c = p & 1;
    const uint32_t a = lds_addr(blk);
    asm volatile(
        "ds_read_b128 %0, %5\n\t"
        "ds_read_b128 %1, %6\n\t"
        "ds_read_b128 %2, %7\n\t"
        "ds_read_b64 %3, %8\n\t"
        "ds_read_b32 %4, %9\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(lo), "=&v"(hi), "=&v"(qh), "=&v"(sc), "=&v"(d)
        : "v"(a + 64u * n + 16u * c), "v"(a + 64u * n + 32u + 16u * c), "v"(a + 128u + 32u * n + 16u * c),
          "v"(a + 192u + 8u * n), "v"(a + 206u)
        : "memory");
}

// Chunks per full segment of a step and DMA instructions per stage.
template <int B, int NSEG>
struct StepGeom {
    static constexpr int kChunksPerSeg = kSB * B / 16;   // 144 (Q4_K) or 210 (Q6_K)
    static constexpr int kChunks = NSEG * kChunksPerSeg;
    static constexpr int kNI = (kChunks + 63) / 64;
    static constexpr int kStageBytes = kNI * 1024;
};

// Per-lane precomputed (segment, chunk) of each of the NI instructions.
template <int B, int NSEG>
struct LaneChunks {
    using G = StepGeom<B, NSEG>;
    int seg[G::kNI];
    int k[G::kNI];
    __device__ __forceinline__ void init(int lane) {
#pragma unroll
        for (int t = 0; t < G::kNI; ++t) {
            const int c = t * 64 + lane;
            const int sg = c / G::kChunksPerSeg;
            seg[t] = sg < NSEG ? sg : NSEG - 1;
            k[t] = sg < NSEG ? c - sg * G::kChunksPerSeg : 0;
        }
    }
};

// Issue the DMA of one step into `slot`.  seg_ptr[j] = first byte of the
// step's part of segment j (16-byte aligned); valid_chunks = chunks present
// in this step (nb_in_step * B / 16).
template <int B, int NSEG>
__device__ __forceinline__ void issue_step(const LaneChunks<B, NSEG>& lc, const uint8_t* const (&seg_ptr)[NSEG],
                                           int valid_chunks, uint8_t* slot) {
    using G = StepGeom<B, NSEG>;
#pragma unroll
    for (int t = 0; t < G::kNI; ++t) {
        const uint8_t* base = seg_ptr[0];
#pragma unroll
        for (int j = 1; j < NSEG; ++j) base = (lc.seg[t] == j) ? seg_ptr[j] : base;
        const int k = lc.k[t] < valid_chunks ? lc.k[t] : 0;
        dma16(base + (size_t)k * 16, slot + t * 1024);
    }
}

}  // namespace rf
