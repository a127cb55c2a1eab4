// Device helpers shared by the LDS-DMA pipelined GEMM kernels (gemm_tiled.hip
// for 16-bit and fp8 inputs, gemm_highp.hip for fp32): the global -> LDS DMA
// load, the vmcnt-bounded workgroup barrier, the A-row LDS swizzle and the
// XCD-aware tile order.
#pragma once

#include "gemm_common.hpp"

#define MB_LDS __attribute__((address_space(3)))

namespace mb {
namespace {

constexpr int kBufferFlags = 0x00020000;  // raw buffer resource word 3 on gfx9

// A-side rows of 64 bytes (4 chunks of 16 bytes): chunk c of row r is stored
// at chunk c ^ swz_a(r), which keeps the 16-byte operand reads of 32
// consecutive rows free of LDS bank conflicts (8- and 16-lane phases).
__device__ __forceinline__ int swz_a(int r) { return ((r >> 1) & 3) ^ ((r >> 3) & 1); }

// Wait until at most N vector-memory operations of this wave are pending and
// its LDS operations have drained, then join the workgroup barrier. The empty
// asm with a memory clobber keeps the compiler from moving LDS accesses
// across the barrier (the barrier builtin alone does not order memory).
template <int N>
__device__ __forceinline__ void wait_vmcnt_and_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
    // gfx9 s_waitcnt encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at [15:14]
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0x0 << 8));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// One LDS-DMA load: every lane fetches 16 bytes at rsrc + voff + soff and the
// wave writes them to LDS bytes [lds_addr, lds_addr + 1024) in lane order.
// Issued as inline asm so the compiler's wait insertion, which cannot tell
// which ring slot the write lands in, does not put a full vmcnt drain in
// front of every later LDS read; the callers order these loads themselves.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rsrc, unsigned lds_addr, int voff, int soff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(lds_addr), "v"(voff), "s"(rsrc), "s"(soff)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// Tile index -> (tile row, tile column). Blocks are dispatched round-robin
// over the 8 XCDs (block b on XCD b % 8); each XCD gets a contiguous range of
// tiles, ordered in groups of `group_m` tile rows, so its concurrent tiles
// form a compact patch whose A and B panels its L2 shares.
__device__ __forceinline__ void tile_coords(int b, int nblocks, int tiles_m, int tiles_n, int group_m,
                                            int* tm, int* tn) {
    int t = b;
    if ((nblocks & 7) == 0) t = (b & 7) * (nblocks >> 3) + (b >> 3);
    const int per_group = group_m * tiles_n;
    const int g = t / per_group;
    const int first_m = g * group_m;
    const int rows = min(tiles_m - first_m, group_m);
    const int r = t - g * per_group;
    *tm = first_m + r % rows;
    *tn = r / rows;
}

}  // namespace
}  // namespace mb
