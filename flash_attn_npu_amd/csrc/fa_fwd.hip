// fa_fwd.hip -- FlashAttention forward for AMD Instinct MI355X (gfx950).
//
// One hand-written HIP kernel family plus the C ABI declared in
// include/fa_fwd.h.  It computes, per (batch, head),
//     O = softmax(sm_scale * Q K^T  [+ causal mask]) V,   LSE = logsumexp(...)
// which is what the reference Triton kernel `_attn_fwd`
// (flash_attention_forward.py:1037-1111, inner loop :648-757, epilogue
// :1022-1033) computes on Ascend.  The work decomposition is gfx950-native:
//
//  * A workgroup owns BM = 32*NW query rows of one (b, h); each of its NW
//    wave64s owns 32 of them.  K and V tiles of BN keys reach LDS by direct
//    DMA (buffer_load ... lds) into a ring of NSTAGE stages, so tile
//    t + NSTAGE - 1 is in flight while tile t is computed and one barrier
//    per tile suffices.
//  * Both products run on v_mfma_f32_32x32x16_{bf16,f16} with fp32
//    accumulation, in transposed form:  S^T = K Q^T  and  O^T = V^T P^T.
//    In the 32x32 accumulator layout lane l holds column l%32, so every lane
//    owns exactly one query: the row max / row sum of the online softmax are
//    in-lane reductions plus one v_permlane32_swap, the rescale factor is a
//    per-lane scalar, and P^T leaves the S^T accumulator already in the
//    B-operand layout of the second MFMA (no LDS round trip for P).
//  * K and V stay row-major in LDS with XOR-swizzled 16-byte chunks; K is
//    read with ds_read_b128 and V^T with the gfx950 transpose read
//    ds_read_b64_tr_b16, so no VGPR or VALU is spent moving or transposing
//    tiles.  With V in fp8-e5m2, P is rounded to e5m2 and O^T = V^T P^T runs
//    on the scaled 32x32x64 fp8 MFMA (V^T read with ds_read_b64_tr_b8).
//  * Q stays in registers for the whole tile loop (AGPRs at D = 256, where
//    one wave per SIMD holds 512 registers).  sm_scale*log2(e) is applied in
//    fp32 after the MFMA (exp2 path); Q is never pre-scaled or re-rounded.
//  * The running max is always kept (numerically stable), with a lazy update:
//    it only moves when a new row max exceeds it by more than 2^8, so the
//    O/l rescale is skipped on most tiles.  Exact by shift invariance.
//  * Causal: KV tiles beyond the workgroup's last query are never loaded,
//    waves skip tiles above their own diagonal, and only tiles crossing the
//    diagonal or the ragged key tail evaluate the mask.  Ragged query/key
//    tails are zero-filled on load, masked to -inf, and never stored.
//  * Workgroups per CU: 2 at D = 128, 1 at D = 256, 3 or 4 at D <= 64, where
//    the softmax VALU work outweighs the MFMAs and more resident waves fill
//    the VALU issue gaps a single wave leaves.
//  * Grid: persistent (as many workgroups as are resident at once); the
//    workgroups of each XCD pull (head, m-tile) tiles, heaviest first, from
//    a tile queue that owns a fixed set of heads, so a head's K/V is read
//    through one L2.  Grids too small to fill the chip split the keys
//    (split-KV) and merge the partial results in a second kernel.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <type_traits>
#include <utility>

#include "fa_fwd.h"
// Host-only planning and the kernel table's metadata (plain C++, also built on
// its own for the host sanitizer test).
#include "fa_plan.cpp"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// The running max only moves when a row max exceeds it by more than this many
// log2 units, so un-normalised probabilities stay <= 2^8 (safe in fp16/bf16).
constexpr float kLazyMaxThreshold = 8.0f;
// Tiles after a unit's first keep the running max while every lane's sum of
// p over the tile (which bounds each of its p) stays within a bound: 2^14
// when P is rounded to fp16 or e5m2 (a quarter of their largest finite
// values), 2^32 for bf16 P (fp32's exponent range; l and O stay far from
// overflow).
template <bool BF16_P>
constexpr float kLazyMaxSum = BF16_P ? 4294967296.0f : 16384.0f;
// FA_TIMING (development builds only): the ping-pong kernel accumulates, per
// wave, the shader-clock cycles spent in each phase and writes them to
// KernelArgs::timing.  The product build compiles none of it.
#ifdef FA_TIMING
#define FA_CLK() ((uint32_t)__builtin_amdgcn_s_memtime())
#define FA_CLK_DELTA(a, b) ((b) - (a))
#endif

struct KernelArgs {
  const char *q;
  const char *k;
  const char *v;
  char *o;
  float *lse;
  int64_t q_sb, q_sh, q_ss;  // element strides (dim stride is 1)
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int32_t B, H, Sq, Sk;
  int32_t n_mtiles;     // ceil(Sq / BM)
  int32_t total_tiles;  // n_mtiles * B * H
  unsigned long long *queue;  // this launch's tile-queue counters (see TileQueue)
  int32_t nq;                 // tile queues: min(8, grid, B*H)
  int32_t q_group;            // heads per group in a queue's order (>= 1)
  int32_t q_bands;            // weight bands in a queue's order (>= 1)
  // Split-KV (DMA kernel only): kv_splits > 1 cuts every m-tile's KV range
  // into runs of split_tiles tiles; each run writes a partial O (fp32,
  // normalised by its own row sum) and its natural-log LSE, and
  // fa_merge_kernel combines them.  kv_splits == 1: O and LSE directly.
  int32_t kv_splits;
  int32_t split_tiles;
  float *part_o;              // [kv_splits][B*H][Sq][D]
  float *part_lse;            // [kv_splits][B*H][Sq]
  uint32_t q_sign;      // 0x80008000 when sm_scale < 0 (Q is negated in registers)
  float c;              // |sm_scale| * log2(e), > 0
  uint32_t *timing;     // per-wave phase cycle counts (FA_TIMING builds only), else null
};

template <bool BF16>
__device__ __forceinline__ f32x16_t mfma32x32x16(u32x4_t a, u32x4_t b, f32x16_t c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                    __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                   __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
}

// Two fp32 -> one dword of two 16-bit values (round to nearest even);
// a single v_cvt_pk_{bf16,f16}_f32 on gfx950.
template <bool BF16>
__device__ __forceinline__ uint32_t pack2(float x, float y) {
  f32x2_t v = {x, y};
  if constexpr (BF16) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
  }
}

// Combine a value across the two lane halves (lane l and lane l^32) with one
// v_permlane32_swap.  The instruction swaps the upper 32 lanes of its first
// operand with the lower 32 lanes of its second; with both operands equal to x
// each lane ends up holding its own value in one result and its partner's in
// the other, so a symmetric op over the two results is the 2-lane reduction.
__device__ __forceinline__ float halves_max(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Buffer resources: one scalar descriptor per (b, h) tensor slice.  Loads
// outside [0, num_records) return zero and stores there are dropped, which is
// how ragged query/key tails are handled without branches.
typedef __amdgpu_buffer_rsrc_t BufRsrc;
constexpr int kBufferFlags = 0x00020000;  // gfx9 dword3: 32-bit data format, no swizzle

__device__ __forceinline__ BufRsrc make_rsrc(const void *base, uint32_t num_bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)num_bytes,
                                           kBufferFlags);
}
__device__ __forceinline__ u32x4_t buf_load16(BufRsrc r, uint32_t voff) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
}
__device__ __forceinline__ void buf_store8(u32x2_t v, BufRsrc r, uint32_t voff) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, voff, 0, 0);
}
__device__ __forceinline__ void buf_store16(u32x4_t v, BufRsrc r, uint32_t voff) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, voff, 0, 0);
}
__device__ __forceinline__ void buf_store4(uint32_t v, BufRsrc r, uint32_t voff) {
  __builtin_amdgcn_raw_buffer_store_b32(v, r, voff, 0, 0);
}

// Position of key `k` (0..BN-1) inside a V^T row in LDS.  In each group of 16
// keys, the 4-key groups 1 and 2 trade places.  This is the order in which a
// lane's S^T accumulator registers reach the B operand of the P*V MFMA: lane
// (h, n) holds keys 8j + 4h + i of a 32-key block in register 4j + i, and
// feeds registers 8t..8t+7 as k-indices 8h..8h+7 of k-step t.
__device__ __forceinline__ int vt_pos(int k) {
  int g = (k >> 2) & 3;
  int pg = (g == 1) ? 2 : (g == 2 ? 1 : g);
  return (k & ~15) | (pg << 2) | (k & 3);
}

// ---------------------------------------------------------------------------
// Tile queues.
//
// Every kernel runs a persistent grid (as many workgroups as are resident at
// once) that pulls (head, m-tile) tiles from nq = min(8, grid, B*H) queues:
// workgroup b serves queue b % nq (the dispatcher sends workgroup b to XCD
// b % 8, so a queue is an XCD's), and queue x owns heads x, x+nq, x+2nq, ...,
// so a head's K/V is only ever read through one XCD's L2.  A queue hands out
// its tiles heaviest first (causal: largest m-tile first, across its heads),
// so the tail is made of the cheapest tiles.  Pulling instead of a static
// split matters on gfx950: workgroups sharing a CU do not progress at the
// same rate (the older one wins issue arbitration), so any fixed assignment
// leaves some of them idle at the end.
//
// Ticket i of a queue is its i-th heaviest tile.  The queue's W workgroups
// take tickets 0..W-1 statically (no atomic before the first tile); later
// tickets come from a counter: ticket = W + atomicAdd(counter, 1), requested
// at the top of a tile so its latency hides behind the tile.  Each of those
// workgroups takes exactly one ticket past the end and stops, so the taker of
// raw count n_tiles - 1 is the last user of the counter and resets it to 0:
// the next launch finds it clean.  The counters live in a device array owned
// by the library, one group of kQueues per launch slot (one 128-byte line per
// counter); launch slots rotate over kQueueSlots, which bounds the eager
// launches that may be in flight on one device.
//
// A launch recorded into a graph (its stream is capturing) gets no counters
// (KernelArgs::queue == nullptr): its workgroups walk the same heaviest-first
// ticket order statically, workgroup w of a queue taking tickets w, w + W,
// w + 2W, ...  Replays of captured launches therefore share no device state
// with each other or with eager launches, whatever streams they run on.
constexpr int kQueues = 8;
constexpr int kQueueSlots = 1024;
constexpr int kQueueStride = 16;  // 128 bytes between counters
__device__ unsigned long long g_tile_queues[kQueueSlots * kQueues * kQueueStride];

struct TileQueue {
  unsigned long long *ctr;  // null: static schedule (graph-captured launch)
  uint32_t n_tiles;   // tiles of this queue
  uint32_t n_static;  // tickets taken without the counter: min(workers, n_tiles)
  uint32_t workers;   // workgroups serving this queue
  int x, nq, nh;      // queue index, queue count, heads of this queue

  __device__ __forceinline__ TileQueue(const KernelArgs &p) {
    nq = p.nq;
    x = blockIdx.x % nq;
    const int BH = p.B * p.H;
    nh = (BH - x + nq - 1) / nq;
    n_tiles = (uint32_t)nh * (uint32_t)p.n_mtiles * (uint32_t)p.kv_splits;
    workers = (gridDim.x - x + nq - 1) / nq;
    n_static = workers < n_tiles ? workers : n_tiles;
    ctr = p.queue != nullptr ? p.queue + x * kQueueStride : nullptr;
  }
  __device__ __forceinline__ uint32_t first() const { return blockIdx.x / nq; }
  __device__ __forceinline__ unsigned long long request() const {
    return ctr != nullptr ? atomicAdd(ctr, 1ull) : 0ull;
  }
  // Ticket of this workgroup's unit it + 1, given the counter value that
  // request() returned during unit it.
  __device__ __forceinline__ uint32_t finish(unsigned long long raw, int it) const {
    if (ctr == nullptr) return first() + (uint32_t)(it + 1) * workers;
    if (raw == n_tiles - 1) atomicExch(ctr, 0ull);
    return n_static + (uint32_t)raw;
  }
  // Ticket -> (head bh, m-tile mt, KV split); false past the end.  Order:
  // KV splits one after the other (split 0 holds the most work); inside a
  // split, the weight ranks k (0 = heaviest m-tile) are cut into `bands`
  // bands; band by band, the queue's heads go in groups of `group`, and
  // inside a group rank-major (heaviest first across the group's heads).
  // Small groups keep a group's K/V in the XCD's L2; bands bound how heavy
  // the last group's tiles are.
  __device__ __forceinline__ bool tile(uint32_t t, int n_mtiles, bool causal, int group, int bands,
                                       int *bh, int *mt, int *split) const {
    if (t >= n_tiles) return false;
    const uint32_t per_split = (uint32_t)nh * (uint32_t)n_mtiles;
    *split = (int)(t / per_split);
    t -= (uint32_t)*split * per_split;
    const int bs = (n_mtiles + bands - 1) / bands;     // ranks per band
    const uint32_t per_band = (uint32_t)nh * (uint32_t)bs;
    const int b = (int)(t / per_band);
    const uint32_t r = t - (uint32_t)b * per_band;
    const int len = min(bs, n_mtiles - b * bs);          // ranks in this band
    const uint32_t per_group = (uint32_t)group * (uint32_t)len;
    const int g = (int)(r / per_group);
    const uint32_t r2 = r - (uint32_t)g * per_group;
    const int gsz = min(group, nh - g * group);          // heads in this group
    const int kk = (int)(r2 / (uint32_t)gsz);
    const int hi = (int)(r2 - (uint32_t)kk * gsz);
    const int k = b * bs + kk;
    *bh = x + nq * (g * group + hi);
    *mt = causal ? n_mtiles - 1 - k : k;
    return true;
  }
};

// ---------------------------------------------------------------------------
// Main kernel: K and V tiles reach LDS by direct DMA (buffer_load ... lds), stay
// row-major there, and are read as MFMA operands with ds_read_b128 (K) and
// the gfx950 transpose read ds_read_b64_tr_b16 (V^T), so no VGPR or VALU is
// spent moving or transposing tiles.  NSTAGE LDS stages form a ring; tile
// t + NSTAGE - 1 is in flight while tile t is computed.
//
// LDS row r (one key, 2*D bytes) stores its 16-byte chunks XOR-swizzled by
// swz<D>(r).  The LDS has 64 banks of 4 bytes (256 bytes per bank row):
//  * D = 128 (256-byte rows, 16 chunks): swz = 4 (r & 3) + ((r >> 2) & 3), a
//    permutation over any 16 consecutive rows, so the 16 lanes of a
//    ds_read_b128 phase (16 consecutive keys, one logical chunk) hit 16
//    distinct bank slots; and for the 4 consecutive rows of a transpose read
//    the high two bits (r & 3) separate their 4-chunk blocks.
//  * D = 256 (512-byte rows): the D = 128 swizzle; only a chunk's position
//    modulo 16 picks its banks, and rows 512 bytes apart align like rows 256
//    bytes apart.
//  * D = 64 (128-byte rows, two per bank row): swz = 4 ((r >> 1) & 1) +
//    ((r >> 2) & 3), a permutation over r >> 1 within each half of the bank
//    row, with rows r and r + 2 of a transpose read in different 4-chunk
//    blocks.
//  * D = 32 (64-byte rows, four per bank row): swz = (r >> 2) & 3 separates
//    rows r, r+4, r+8, r+12 of a ds_read_b128 phase.
//  * D = 16 (32-byte rows, eight per bank row): swz = (r >> 3) & 1 separates
//    rows r and r+8.
// Every DMA instruction still writes 1 KB contiguously and reads whole rows
// from HBM.
template <int D>
__device__ __forceinline__ int swz(int r) {
  if constexpr (D == 128 || D == 256) {
    return ((r & 3) << 2) | ((r >> 2) & 3);
  } else if constexpr (D == 64) {
    return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
  } else if constexpr (D == 32) {
    return (r >> 2) & 3;
  } else {
    static_assert(D == 16, "head dim");
    return (r >> 3) & 1;
  }
}

// Chunk swizzle of fp8-e5m2 V rows (D bytes), read with ds_read_b64_tr_b8.
// One read's half-wave touches rows {0..3, 8..11} of a 16-key step (+4 in
// the upper half-wave), 8 bytes in each of two adjacent chunks per row:
//  * D = 256 (a row is one 256-byte bank row): the eight rows get distinct
//    even chunk offsets, 2 ((r & 3) + 4 ((r >> 3) & 1));
//  * D = 128 (two rows per bank row): the four rows of one parity get
//    distinct even chunk offsets, 2 ((r >> 1) & 1) + 4 ((r >> 3) & 1);
//  * D = 64 (four rows per bank row): rows r and r + 8 differ by 2 chunks.
//  * D = 32 (eight rows per bank row): rows r and r + 8 share their banks
//    whatever the chunk order, so the read takes two passes; no swizzle;
//  * D = 16: one chunk per row, no swizzle (rows 0..15 fill a bank row).
template <int D>
__device__ __forceinline__ int swz8(int r) {
  if constexpr (D == 256) {
    return ((r & 3) | (((r >> 3) & 1) << 2)) << 1;
  } else if constexpr (D == 128) {
    return (((r >> 1) & 1) << 1) | (((r >> 3) & 1) << 2);
  } else if constexpr (D == 64) {
    return ((r >> 3) & 1) << 1;
  } else {
    static_assert(D == 32 || D == 16, "fp8 V head dim");
    return 0;
  }
}

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) char lds_char;

__device__ __forceinline__ u32x2_t lds_read_tr16(const char *smem_base, uint32_t off) {
  const lds_char *p = (const lds_char *)smem_base + off;
  i16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4_t *)p);
  return __builtin_bit_cast(u32x2_t, v);
}

// Transposing 8-bit read (ds_read_b64_tr_b8): in each group of 16 lanes,
// output lane i receives, as byte j of its 8 bytes, byte (i % 8) of the
// 8 bytes addressed by lane 2j + i/8 of the group.
__device__ __forceinline__ u32x2_t lds_read_tr8(const char *smem_base, uint32_t off) {
  const lds_char *p = (const lds_char *)smem_base + off;
  typedef int i32x2_t __attribute__((ext_vector_type(2)));
  i32x2_t v = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) i32x2_t *)p);
  return __builtin_bit_cast(u32x2_t, v);
}

// One 16-byte-per-lane DMA: lane i writes LDS bytes [lds + 16 i, +16) with
// the buffer bytes at voff (out-of-range reads give zeros).  Issued as inline
// asm so the compiler does not treat later LDS reads as aliasing the
// in-flight DMA (it would insert vmcnt(0) before them and serialise the
// prefetch); completion is enforced explicitly with s_waitcnt vmcnt + barrier
// before a stage is read.  M0 carries the LDS base and is set right here.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(BufRsrc r, uint32_t lds_addr, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voff), "s"(r)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// The same DMA through the compiler builtin: the compiler sees it as a
// buffer load (so sched_group_barrier can place it between MFMAs) and, when
// the LDS target is a different __shared__ array from the one being read,
// adds no wait in front of those reads.
__device__ __forceinline__ void dma16_lds(BufRsrc r, char *lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)(lds_char *)lds, 16, voff, 0,
                                           0, 0);
}

// s_waitcnt immediate: vmcnt(n), no wait on expcnt / lgkmcnt.
constexpr int vmcnt_imm(int n) { return 0x0f70 | (n & 0xf) | ((n >> 4) << 14); }

// sched_group_barrier masks.
constexpr int kSchedVmem = 0x010;
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;

template <int D, int BN, int NW, int NSTAGE, int OCC, bool V8 = false>
struct Cfg2 {
  static constexpr int BM = 32 * NW;
  static constexpr int NT = 64 * NW;
  static constexpr int ROW = 2 * D;           // bytes per K row in LDS
  static constexpr int CPR = ROW / 16;        // 16-byte chunks per row
  static constexpr int RPI = 1024 / ROW;      // rows per DMA instruction (64 lanes x 16 B)
  static constexpr int TILE = BN * ROW;       // bytes of one K tile
  static constexpr int IPT = TILE / 1024;     // DMA instructions per K tile
  static constexpr int IPW = IPT / NW;        // ... per wave
  // V rows: D 16-bit elements, or D bytes when V is fp8-e5m2 (V8).
  static constexpr int VROW = V8 ? D : 2 * D;
  static constexpr int VCPR = VROW / 16;
  static constexpr int VRPI = 1024 / VROW;
  static constexpr int VTILE = BN * VROW;
  static constexpr int VIPT = VTILE / 1024;
  // An fp8 V tile of D <= 32 is less than one DMA instruction per wave: every
  // wave still issues one, the extra waves fetch the rows after the tile
  // (in range, or zeros past Sk) into LDS padding that is never read.
  static constexpr int VIPW = VIPT >= NW ? VIPT / NW : 1;
  static constexpr int VTILE_LDS = VIPW * NW * 1024;
  static constexpr int NDMA = IPW + VIPW;     // DMA instructions per wave and tile
  static constexpr int STAGE = TILE + VTILE_LDS;
  // One workgroup per CU, 16-bit V, and fewer DMA chunks per wave than 32 Q
  // rows fill (the 32-key D = 256 kernels): Q comes in through an LDS area of
  // its own, BM rows of 2 D bytes.
  static constexpr bool QAREA = OCC == 1 && !V8 && NDMA < D / 16;
  static constexpr int Q_BYTES = QAREA ? BM * 2 * D : 0;
  static constexpr int LDS_BYTES = NSTAGE * STAGE + Q_BYTES;
  // O^T blocks of 32 head dims; D = 16 uses one block whose upper 16 rows
  // come out zero (the V^T operand rows past D are zeroed).
  static constexpr int DB = D >= 32 ? D / 32 : 1;
  static_assert(D == 16 || D == 32 || D == 64 || D == 128 || D == 256, "head dim");
  static_assert(IPT % NW == 0 && IPW >= 1, "DMA instructions must split evenly over waves");
  static_assert(VIPT % NW == 0 || (V8 && VIPT < NW), "DMA instructions must split evenly over waves");
  static_assert(!V8 || (BN % 64 == 0 && (D >= 32 ? BN == 64 : BN == 128)), "fp8 V: 64-key tiles (D = 16: 128)");
  static_assert(BN % 32 == 0, "tile shape");
  static_assert(NSTAGE == 2, "double-buffered: one tile computes while the next lands");
  static_assert(OCC >= 1 && OCC <= 4, "workgroups per CU");
  static_assert(LDS_BYTES * OCC <= 160 * 1024, "LDS budget of one gfx950 CU");
};

// V8: V is fp8-e5m2 (reference flash_attention_forward.py:704, :737, :996):
// P is rounded to e5m2 and O^T += V^T P^T runs on the 32x32x64 fp8 MFMA, one
// instruction per 32 head dims and 64 keys.  Q, K and O keep their 16-bit type.
template <int D, int BN, int NW, int NSTAGE, int OCC, bool BF16, bool CAUSAL, bool V8 = false>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(OCC * NW / 4, OCC * NW / 4)))
fa_fwd_dma_kernel(KernelArgs p) {
  using C = Cfg2<D, BN, NW, NSTAGE, OCC, V8>;
  constexpr int ESV = V8 ? 1 : 2;  // bytes per V element
  // fp16 at D = 16, where the softmax VALU work dwarfs the 12 MFMAs of a
  // tile: the row sum moves from BN VALU adds per tile to BN / 16 MFMAs over
  // the fp16 P (relative change of l at most 2^-11, the fp16 rounding of p;
  // bf16 would allow 2^-9, too close to the LSE tolerance).  Measured 5.6%
  // faster at D = 16; at D = 32 equal and at D = 64 1.3-1.8% slower, where
  // the extra MFMA time costs what the adds saved.
  constexpr bool MSUM = !BF16 && !V8 && D == 16;
  // Tiles after a unit's first take the row max only when p outgrows 2^8
  // (see the tile body); the kept scores then cost D * BN / 64 more live
  // registers, which the kernels with 128-key tiles, 64-key D = 256 tiles or
  // the 168-register budget of three D = 128 workgroups per CU cannot spare
  // (they spill): those take the row max of every tile.
  constexpr bool kSumTrigger = !MSUM && BN <= 64 && D * BN <= 8192 && !(D >= 128 && OCC >= 3);
  constexpr int BM = C::BM;
  // One array per stage: the compiler's LDS-DMA alias tracking then knows
  // that DMAs into one stage never feed reads of the other, and adds no
  // vmcnt wait in front of them.
  __shared__ __attribute__((aligned(1024))) char smem0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char smem1[C::STAGE];
  // Q area (C::QAREA kernels only): the launch's dynamic LDS, which follows
  // the static arrays, so the stages stay in the low 64 KB where every K and
  // V^T read is a per-lane base plus an immediate offset (a static area was
  // placed first and cost the kernel 58 registers of addresses).  Wave w's Q
  // rows take bytes [32 w, 32 w + 32) x 2 D.  (Staging O there as well, in one
  // pass instead of two through the stages, measured no faster.)
  extern __shared__ __attribute__((aligned(1024))) char smemq[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31;
  const int h = lane >> 5;

  // DMA: instruction j of this wave fills LDS rows (wave + j*NW)*RPI .. +RPI of
  // the tile; lane -> (row, physical chunk), and it fetches the logical chunk
  // that the swizzle stores there.
  uint32_t dk[C::IPW], dv[C::VIPW];
#pragma unroll
  for (int j = 0; j < C::IPW; ++j) {
    const int row = (wave + j * NW) * C::RPI + lane / C::CPR;
    const int lc = (lane % C::CPR) ^ swz<D>(row);
    dk[j] = (uint32_t)(row * p.k_ss * 2 + lc * 16);
  }
#pragma unroll
  for (int j = 0; j < C::VIPW; ++j) {
    const int row = (wave + j * NW) * C::VRPI + lane / C::VCPR;
    int lc = lane % C::VCPR;
    if constexpr (V8)
      lc ^= swz8<D>(row);
    else
      lc ^= swz<D>(row);
    dv[j] = (uint32_t)(row * p.v_ss * ESV + lc * 16);
  }
  // K operand reads: lane (h, n) reads key row 32kb + n, logical chunk 2s + h
  // (swz(32kb + n) == swz(n)).
  uint32_t kro[D / 16];
#pragma unroll
  for (int s = 0; s < D / 16; ++s) kro[s] = (uint32_t)(n * C::ROW + (((2 * s + h) ^ swz<D>(n)) * 16));
  // V^T operand reads (transpose): in lane group g = lane/16, source lane
  // 4j + c points at key row 16ks + 8e + 4h + j, dims 32db + 16(g&1) + 4c
  // (logical chunk 4db + 2(g&1) + c/2).  swz of that row depends only on
  // (e, h, j), so one lane offset per (db, e) covers every k-step ks.
  // D = 16: lanes of the upper 16 dims read dims 0..15 again (in range) and
  // their fragments are zeroed before use.
  //
  // fp8 V (8-bit transpose reads, one per 16 keys): the fp8 MFMA pairs byte
  // j of lane half h of both operands; P^T takes byte j from S^T register
  // (block j / 16, r = j % 16), i.e. key 16 (j / 8) + 8 ((j % 8) >> 2) + 4h +
  // (j & 3).  So for the read of key step u (bytes 8u..8u+7), source lane s
  // of lane group g = lane/16 addresses key row 16u + 8 ((s >> 1) >> 2) +
  // 4 (g >> 1) + ((s >> 1) & 3), dims 32db + 16 (g & 1) + 8 (s & 1); the
  // swizzle of that row does not depend on u.
  uint32_t vro[C::DB][V8 ? 1 : 2];
  if constexpr (V8) {
    const int g = lane >> 4, sl = lane & 15, q = sl >> 1;
    const int row = 8 * (q >> 2) + 4 * (g >> 1) + (q & 3);
#pragma unroll
    for (int db = 0; db < C::DB; ++db) {
      // D = 16: lanes of the upper 16 dims re-read dims 0..15 (in the row)
      // and their fragments are zeroed before use.
      const int lc = 2 * db + (D >= 32 ? (g & 1) : 0);
      vro[db][0] = (uint32_t)(row * C::VROW + ((lc ^ swz8<D>(row)) * 16) + (sl & 1) * 8);
    }
  } else {
    const int g = lane >> 4, sg = lane & 15, jj = sg >> 2, cc = sg & 3;
#pragma unroll
    for (int db = 0; db < C::DB; ++db)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int row = 8 * e + 4 * h + jj;
        const int lc = 4 * db + (D >= 32 ? 2 * (g & 1) : 0) + (cc >> 1);
        vro[db][e] = (uint32_t)((4 * h + jj) * C::ROW + ((lc ^ swz<D>(row)) * 16) + (cc & 1) * 8);
      }
  }

  const float c = p.c;

  // Tile loop: thread 0 takes tickets (the next one is requested at the top
  // of a tile and published through LDS at its end, behind a barrier).
  __shared__ uint32_t s_ticket[2];
  const TileQueue tq(p);
  int bh, mt, split;
  for (int it = 0; tq.tile(it == 0 ? tq.first() : s_ticket[it & 1], p.n_mtiles, CAUSAL, p.q_group, p.q_bands,
                           &bh, &mt, &split);
       ++it) {
    unsigned long long next_raw = 0;
#ifdef FA_TIMING
    uint32_t tm_vm = 0, tm_bar = 0, tm_cmp = 0, n_comp = 0, tm_pro = 0, tm_epi0 = 0, tm_dma = 0, tm_idle = 0;
    const uint32_t tm0 = FA_CLK();
    const uint32_t rt0 = (uint32_t)__builtin_amdgcn_s_memrealtime();
#endif
    const int bb = bh / p.H;
    const int hh = bh - bb * p.H;

    const int q0 = mt * BM;
    const int q0w = q0 + 32 * wave;
    const int qrow = q0w + n;

    const char *qg = p.q + 2 * (bb * p.q_sb + hh * p.q_sh);
    const char *kg = p.k + 2 * (bb * p.k_sb + hh * p.k_sh);
    const char *vg = p.v + ESV * (bb * p.v_sb + hh * p.v_sh);

    const int kv_end = CAUSAL ? min(p.Sk, q0 + BM) : p.Sk;
    // KV tiles [t_begin, n_tiles) of this unit: the whole range, or one run
    // of split_tiles tiles under split-KV (possibly empty past the diagonal).
    const int t_begin = split * p.split_tiles;
    const int n_tiles = min((kv_end + BN - 1) / BN, t_begin + p.split_tiles);
    const int wave_last_q = q0w + 31;
    // Thread 0 takes the next ticket.  When wave 0 has no work in the unit's
    // last tile (under the causal mask its rows end before that tile's keys,
    // or they lie past Sq), the request waits for that idle tile: the atomic
    // returns while the other waves compute it, and units start in ticket
    // order.  Requested at the unit's start, a ticket stayed reserved for a
    // whole unit and heavy units taken that way started late (B4 H32 S2048
    // causal: the workgroups of one queue ended between 114 and 144 us).
    // Otherwise (every wave computes the last tile; non-causal units are all
    // alike anyway) it is requested at the unit's start, where its latency
    // hides behind the first tile's loads; a request inside the tile code
    // cost the kernels 30 or more registers.
    // Tiles visible to every query of the workgroup (no mask needed).
    auto n_full_of = [&](int q0_) __attribute__((always_inline)) {
      int nf = p.Sk / BN;
      if (CAUSAL) nf = min(nf, (q0_ + 1) / BN);
      return min(nf, n_tiles);
    };
    const int t_last = n_tiles - 1;
    const int w0_act = (CAUSAL && OCC >= 2) ? max(n_full_of(q0), min(n_tiles, (q0 + 31) / BN + 1)) : n_tiles;
    const bool late_ticket = OCC >= 2 && n_tiles > t_begin && (q0 >= p.Sq || w0_act < n_tiles);
    if (threadIdx.x == 0 && !late_ticket) next_raw = tq.request();

    // DMA of KV tile t into stage STG: instruction i < 2*IPW of this wave
    // (K rows for even i, V rows for odd i).  Past the last tile the buffer
    // range is empty: the instructions still issue (so the same code covers
    // every tile) but fetch nothing and write zeros into the free stage.
    auto tile_rsrc = [&](int t, BufRsrc *rk, BufRsrc *rv) __attribute__((always_inline)) {
      const int key0 = t * BN;
      const bool live = t < n_tiles;
      const uint32_t nbk = live ? (uint32_t)((int64_t)(p.Sk - key0) * p.k_ss * 2) : 0u;
      const uint32_t nbv = live ? (uint32_t)((int64_t)(p.Sk - key0) * p.v_ss * ESV) : 0u;
      *rk = make_rsrc(kg + (int64_t)key0 * p.k_ss * 2, nbk);
      *rv = make_rsrc(vg + (int64_t)key0 * p.v_ss * ESV, nbv);
    };
    // With fp8 V the K instructions come first, then the (fewer) V ones.
    auto dma = [&](auto stage_tag, const BufRsrc &rk, const BufRsrc &rv, int i) __attribute__((always_inline)) {
      constexpr int STG = decltype(stage_tag)::value;
      char *base = STG == 0 ? smem0 : smem1;
      if constexpr (V8) {
        if (i < C::IPW)
          dma16_lds(rk, base + (wave + i * NW) * 1024, dk[i]);
        else
          dma16_lds(rv, base + C::TILE + (wave + (i - C::IPW) * NW) * 1024, dv[i - C::IPW]);
      } else {
        const int j = i >> 1;
        dma16_lds((i & 1) ? rv : rk, base + (i & 1) * C::TILE + (wave + j * NW) * 1024, (i & 1) ? dv[j] : dk[j]);
      }
    };

    // Prologue: KV tile t_begin into its stage (t_begin & 1), and this wave's
    // Q rows.
    auto kv_prologue = [&](auto stage_tag) __attribute__((always_inline)) {
      BufRsrc rk, rv;
      tile_rsrc(t_begin, &rk, &rv);
#pragma unroll
      for (int i = 0; i < C::NDMA; ++i) dma(stage_tag, rk, rv, i);
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    u32x4_t qf[D / 16];
    {
      const BufRsrc rq = make_rsrc(qg, (uint32_t)((int64_t)p.Sq * p.q_ss * 2));
      // A lane's Q fragment s is 16 bytes of its own row (bytes 32s + 16h),
      // so loading fragments directly makes every load instruction touch 32
      // rows.  Where the 1 KB LDS chunks that this wave's DMAs fill hold its
      // 32 rows, Q comes through them instead: DMAs that each read 1 KB of
      // whole rows, into the stage that tile t_begin does not use (free until
      // the first tile's DMAs, which this wave issues after the reads below
      // have completed; other waves' DMAs fill only their own chunks), then
      // one LDS read per fragment.  16-byte units of a row sit XOR-swizzled
      // by the row, so the 32 rows of a read spread over the banks.  The Q
      // DMAs go first so that waiting for them leaves the K/V DMAs in flight
      // (vmcnt retires in issue order).  At three or more workgroups per CU
      // the others hide a unit's prologue and the staging measured 1% slower
      // (B16 H16 S1024 D64), so those kernels load Q directly.  The 32-key
      // D = 256 kernels, whose chunks hold 16 rows, stage Q the same way
      // through a Q area of their own (0.2-0.9% faster than direct loads),
      // and the fp8-V D = 256 kernel, whose stages leave no room for one,
      // loads it directly.
      constexpr bool kQOwn = C::NDMA >= D / 16 && OCC <= 2;
      static_assert(!(kQOwn && C::QAREA), "one Q staging area");
      constexpr int W = 2 * D;                                 // bytes per row
      constexpr int RPC = 1024 / W;                            // rows per chunk
      constexpr int U = W / 16;                                // 16-byte units per row
      constexpr int USW = U < 32 ? U : 32;                     // swizzle span
      // Q rows of this wave into 1 KB chunks chunk(k) (k < 32 / RPC), the
      // K/V DMAs of tile t_begin behind them, then the fragments from LDS.
      auto q_staged = [&](auto chunk, int ln, auto kv_tag) __attribute__((always_inline)) {
        const int rr = ln / U, slot = ln % U;
#pragma unroll
        for (int k = 0; k < 32 / RPC; ++k) {  // chunk k: rows k RPC .. + RPC, lane -> (row, slot)
          const int row = k * RPC + rr;
          dma16_lds(rq, chunk(k), (uint32_t)((q0w + row) * p.q_ss * 2 + ((slot ^ (row & (USW - 1))) << 4)));
        }
        kv_prologue(kv_tag);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(C::NDMA));
        const int ln_n = ln & 31, ln_h = ln >> 5;
        const char *const rb = chunk(ln_n / RPC) + (ln_n % RPC) * W;
        const int sw = ln_n & (USW - 1);
#pragma unroll
        for (int s = 0; s < D / 16; ++s) qf[s] = *(const u32x4_t *)(rb + (((2 * s + ln_h) ^ sw) << 4)) ^ p.q_sign;
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): reads done before the chunks take DMAs again
      };
      if constexpr (kQOwn) {
        int ln = lane, wv = wave;  // opaque: keeps the addresses in the prologue
        asm volatile("" : "+v"(ln), "+s"(wv));
        auto run_q = [&](auto q_tag, auto kv_tag) __attribute__((always_inline)) {
          char *const qb = decltype(q_tag)::value == 0 ? smem0 : smem1;
          auto chunk = [&](int k) __attribute__((always_inline)) {
            return qb + (k < C::IPW ? (wv + k * NW) * 1024 : C::TILE + (wv + (k - C::IPW) * NW) * 1024);
          };
          q_staged(chunk, ln, kv_tag);
        };
        if (t_begin & 1)
          run_q(S0{}, S1{});
        else
          run_q(S1{}, S0{});
      } else if constexpr (C::QAREA) {
        // The wave's 32 rows in its own part of the Q area: nothing else
        // writes there, and its next accesses to it follow these reads.
        int ln = lane, wv = wave;  // opaque: keeps the addresses in the prologue
        asm volatile("" : "+v"(ln), "+s"(wv));
        char *const qb = smemq + wv * (32 * W);
        auto chunk = [&](int k) __attribute__((always_inline)) { return qb + k * 1024; };
        if (t_begin & 1)
          q_staged(chunk, ln, S1{});
        else
          q_staged(chunk, ln, S0{});
      } else {
        if (t_begin & 1)
          kv_prologue(S1{});
        else
          kv_prologue(S0{});
        const uint32_t qo = (uint32_t)(qrow * p.q_ss * 2 + 16 * h);
#pragma unroll
        for (int s = 0; s < D / 16; ++s) qf[s] = buf_load16(rq, qo + 32 * s) ^ p.q_sign;
      }
      // One workgroup per CU (D = 256, 16-bit V): Q lives in AGPRs (the MFMA
      // reads its B operand from there), which leaves the VGPRs to S, P and the
      // fragments.  (With fp8 V the 64-key S block takes those AGPRs.)
      if constexpr (OCC == 1 && !V8) {
#pragma unroll
        for (int s = 0; s < D / 16; ++s) asm volatile("" : "+a"(qf[s]));
      }
    }

    f32x16_t oacc[C::DB];
#pragma unroll
    for (int db = 0; db < C::DB; ++db) oacc[db] = (f32x16_t){};
    float m_run = -INFINITY;
    float l_run = 0.f;
    // MSUM: the row sum l on the matrix core, as one more O^T block whose
    // A operand is 1 in rows 0 and 4 (lane halves' element 0) and 0 elsewhere:
    // l = sum of the fp16 P fed to P.V, in fp32.
    f32x16_t lacc = {};
    const uint32_t one2 = ((lane & 31) == 0 || (lane & 31) == 4) ? 0x3C003C00u : 0u;  // fp16 (1, 1)
    const u32x4_t ones = {one2, one2, one2, one2};

    // One KV tile: wait for its DMA, barrier, refill the other stage, then
    // S^T = K Q^T, online softmax, O^T += V^T P^T.  MASKED is a compile-time
    // switch: only tiles crossing the diagonal or the ragged key tail pay for
    // the mask (and for skipping tiles above a wave's own rows), and neither
    // loop body branches on it.  STG = t % 2 is compile-time too, so every
    // LDS read address is a per-lane base plus an immediate offset.
    auto kv_tile = [&](int t, auto masked_tag, auto stage_tag, auto exact_tag,
                       auto half_tag) __attribute__((always_inline)) {
      constexpr bool MASKED = decltype(masked_tag)::value;
      constexpr int STG = decltype(stage_tag)::value;
      constexpr bool EXACT = decltype(exact_tag)::value;  // the unit's first tile
      // Tiles after the first of 64 keys (16-bit V) take the block-split body.
      constexpr bool SPLIT = kSumTrigger && !EXACT && !V8 && BN == 64;
      // HALF: a masked tile whose second 32-key block lies past every row of
      // this wave (causal), so only the first block is computed.
      constexpr bool HALF = decltype(half_tag)::value;
      static_assert(!HALF || (SPLIT && MASKED), "half tiles take the block-split masked body");
#ifdef FA_TIMING
      const uint32_t ta = FA_CLK();
      if (t == 0) tm_pro = ta - tm0;
#endif
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
#ifdef FA_TIMING
      const uint32_t tb = FA_CLK();
#endif
      __syncthreads();
#ifdef FA_TIMING
      const uint32_t tc = FA_CLK();
      tm_vm += tb - ta;
      tm_bar += tc - tb;
#endif
      // The next tile's DMAs go into the other stage (free after the
      // barrier); they are spread over the QK MFMAs below, or issued here
      // when this wave has no work in this tile.
      constexpr int NDMA = C::NDMA;
      using NEXT = std::integral_constant<int, 1 - STG>;
      BufRsrc rk_n, rv_n;
      tile_rsrc(t + 1, &rk_n, &rv_n);
#ifdef FA_TIMING
      const uint32_t td = FA_CLK();
      tm_dma += td - tc;
#endif

      const int kbase = t * BN;
#ifdef FA_TIMING
      ++n_comp;
      struct Stamp {
        uint32_t &acc, t0;
        __device__ ~Stamp() { acc += FA_CLK() - t0; }
      } stamp{tm_cmp, FA_CLK()};
#endif

      const char *sbase = STG == 0 ? smem0 : smem1;

      // S^T = K Q^T.  Fragment i = (s, kb); K fragments are read KPF ahead of
      // their MFMA, the next tile's DMAs go out one per MFMA, and the first
      // VPF V^T fragments of the P*V product are issued right behind the K
      // reads so they land during the softmax.
      constexpr int NQK = (D / 16) * (BN / 32);
      // K fragments read KPF MFMAs ahead (3 in the three-workgroups-per-CU
      // D = 128 kernel, whose 168 registers hold no fourth fragment without
      // spilling).
      constexpr int KPF = (OCC >= 3 && D == 128) ? 3 : 4;
      constexpr int NPV = V8 ? (BN / 64) * C::DB : (BN / 16) * C::DB;
      constexpr int VPF = V8 ? 1 : 2;
      constexpr int VRD = V8 ? 4 : 2;  // LDS reads per V^T fragment
      // fp8 V^T fragment i = (64-key chunk kc, head dims 32db..): 32 bytes per lane.
      auto vread8 = [&](int i) {
        const int kc = i / C::DB, db = i % C::DB;
        i32x8_t f;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const u32x2_t x = lds_read_tr8(sbase, vro[db][0] + (uint32_t)(C::TILE + (64 * kc + 16 * u) * C::VROW));
          f[2 * u] = (int)x[0];
          f[2 * u + 1] = (int)x[1];
        }
        if constexpr (D < 32) {
          if (lane & 16) f = (i32x8_t){0, 0, 0, 0, 0, 0, 0, 0};
        }
        return f;
      };
      auto vread = [&](int i) {
        const int ks = i / C::DB, db = i % C::DB;
        const uint32_t imm = (uint32_t)(C::TILE + 16 * ks * C::ROW);
        const u32x2_t lo = lds_read_tr16(sbase, vro[db][0] + imm);
        const u32x2_t hi = lds_read_tr16(sbase, vro[db][V8 ? 0 : 1] + imm + 8 * C::ROW);
        u32x4_t f = {lo[0], lo[1], hi[0], hi[1]};
        if constexpr (D < 32) {
          if (lane & 16) f = (u32x4_t){0u, 0u, 0u, 0u};
        }
        return f;
      };
      u32x4_t kfr[NQK];
      u32x4_t vfr[V8 ? 1 : NPV];
      i32x8_t vfr8[V8 ? NPV : 1];
      f32x16_t sacc[BN / 32];
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb) sacc[kb] = (f32x16_t){};
      // p = 2^(s c - mb) per 32-key block.
      f32x16_t pacc[BN / 32];
      auto rescale = [&](float alpha) __attribute__((always_inline)) {
        if constexpr (MSUM)
          lacc[0] *= alpha;
        else
          l_run *= alpha;
#pragma unroll
        for (int db = 0; db < C::DB; ++db) oacc[db] *= alpha;
      };
      // Register r of block kb holds key kbase + 4h + (32kb + 8(r>>2) + (r&3));
      // it is visible iff that offset <= lim.
      auto mask_block = [&](int kb) __attribute__((always_inline)) {
        const int last_key = CAUSAL ? min(qrow, p.Sk - 1) : p.Sk - 1;
        const int lim = last_key - kbase - 4 * h;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int off = 32 * kb + 8 * (r >> 2) + (r & 3);
          sacc[kb][r] = off <= lim ? sacc[kb][r] : -INFINITY;
        }
      };

      if constexpr (SPLIT) {
        // Two 32-key blocks, each carried through on its own: the QK MFMAs
        // run block by block, block 0's exponentials issue between block 1's
        // QK MFMAs, and block 1's between block 0's P.V MFMAs, so the wave
        // keeps the matrix core busy through most of its own softmax.  The
        // running max is handled per block as in the whole-tile form (it
        // moves only when a block's lane sum exceeds kLazyMaxSum; O and l,
        // including block 0's P.V, are then rescaled): exact by shift
        // invariance.
        constexpr int NS = D / 16;  // k-steps per block
        auto kread_b = [&](int i) {
          const int kb = i / NS, s = i % NS;
          return *(const u32x4_t *)(sbase + kro[s] + 32 * kb * C::ROW);
        };
        float bpart[2];
        auto exps_block = [&](int kb, float m) __attribute__((always_inline)) {
          const float mb = (m == -INFINITY) ? 0.f : m;
          float lsum[4];
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float pv = fast_exp2(__builtin_fmaf(sacc[kb][r], c, -mb));
            pacc[kb][r] = pv;
            lsum[r & 3] = r < 4 ? pv : lsum[r & 3] + pv;
          }
          bpart[kb] = (lsum[0] + lsum[1]) + (lsum[2] + lsum[3]);
        };
        auto settle_block = [&](int kb) __attribute__((always_inline)) {
          if (__builtin_amdgcn_ballot_w64(!(bpart[kb] <= kLazyMaxSum<BF16 && !V8>))) {
            float mx = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kb][r]);
            const float m_new = fmaxf(m_run, halves_max(mx) * c);
            rescale(m_new == m_run ? 1.f : fast_exp2(m_run - m_new));
            m_run = m_new;
            exps_block(kb, m_run);
          }
          l_run += bpart[kb];
        };
        u32x4_t pf[4];
        auto pack_block = [&](int kb) __attribute__((always_inline)) {
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int w = 0; w < 4; ++w)
              pf[2 * kb + u][w] = pack2<BF16>(pacc[kb][8 * u + 2 * w], pacc[kb][8 * u + 2 * w + 1]);
        };
        // Number of softmax VALU instructions placed after each MFMA.
        constexpr int kValuPerMfma = 7;
        constexpr int kSchedValu = 0x002 | 0x400;  // VALU and TRANS
        constexpr int NPVB = 2 * C::DB;  // P.V MFMAs per block

        if constexpr (HALF) {
          // Block 1 is masked for every row of the wave: its p are 0 and it
          // adds nothing to l or O, so block 0 alone gives the same result.
          // The tile's DMAs still go out, one per QK MFMA.
          static_assert(C::NDMA <= NS, "one DMA per QK MFMA of block 0");
          constexpr int VAT = NS - 1;  // V^T reads at the last QK step (fewer live fragments)
#pragma unroll
          for (int i = 0; i < KPF && i < NS; ++i) kfr[i] = kread_b(i);
#pragma unroll
          for (int i = 0; i < NS; ++i) {
            if (i + KPF < NS) kfr[i + KPF] = kread_b(i + KPF);
            if (i == VAT) {
#pragma unroll
              for (int j = 0; j < VPF; ++j) vfr[j] = vread(j);
            }
            sacc[0] = mfma32x32x16<BF16>(kfr[i], qf[i], sacc[0]);
            if (i < NDMA) dma(NEXT{}, rk_n, rv_n, i);
          }
          mask_block(0);
          exps_block(0, m_run);
          settle_block(0);
          if constexpr (D >= 128) __builtin_amdgcn_s_setprio(1);
          pack_block(0);
#pragma unroll
          for (int i = 0; i < NPVB; ++i) {
            if (i + VPF < NPVB) vfr[i + VPF] = vread(i + VPF);
            const int ks = i / C::DB, db = i % C::DB;
            oacc[db] = mfma32x32x16<BF16>(vfr[i], pf[ks], oacc[db]);
          }
          if constexpr (D >= 128) __builtin_amdgcn_s_setprio(0);
          return;
        }

        // S^T = K Q^T block by block (reads KPF ahead, one DMA per MFMA),
        // block 0's softmax under block 1's MFMAs.
#pragma unroll
        for (int i = 0; i < KPF; ++i) kfr[i] = kread_b(i);
#pragma unroll
        for (int i = 0; i < NQK; ++i) {
          if (i + KPF < NQK) kfr[i + KPF] = kread_b(i + KPF);
          if (i + KPF == NQK) {
#pragma unroll
            for (int j = 0; j < VPF; ++j) vfr[j] = vread(j);
          }
          const int kb = i / NS, s = i % NS;
          sacc[kb] = mfma32x32x16<BF16>(kfr[i], qf[s], sacc[kb]);
          if (i < NDMA) dma(NEXT{}, rk_n, rv_n, i);
        }
        if (MASKED) mask_block(0);
        exps_block(0, m_run);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, KPF, 0);
#pragma unroll
        for (int i = 0; i < NQK; ++i) {
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
          if (i < NDMA) __builtin_amdgcn_sched_group_barrier(kSchedVmem, 1, 0);
          if (i + KPF < NQK) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
          if (i + KPF == NQK) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, VRD * VPF, 0);
          if (i >= NS) __builtin_amdgcn_sched_group_barrier(kSchedValu, kValuPerMfma, 0);
        }
        settle_block(0);

        // O^T += V^T P^T for block 0's keys (k-steps 0, 1) with block 1's
        // softmax between the MFMAs, then block 1's keys.
        if constexpr (D >= 128) __builtin_amdgcn_s_setprio(1);
        pack_block(0);
#pragma unroll
        for (int i = 0; i < NPVB; ++i) {
          vfr[i + VPF] = vread(i + VPF);
          const int ks = i / C::DB, db = i % C::DB;
          oacc[db] = mfma32x32x16<BF16>(vfr[i], pf[ks], oacc[db]);
        }
        if (MASKED) mask_block(1);
        exps_block(1, m_run);
        __builtin_amdgcn_sched_group_barrier(kSchedValu, 8, 0);  // block 0's packs
#pragma unroll
        for (int i = 0; i < NPVB; ++i) {
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedValu, kValuPerMfma, 0);
        }
        settle_block(1);
        pack_block(1);
#pragma unroll
        for (int i = NPVB; i < NPV; ++i) {
          if (i + VPF < NPV) vfr[i + VPF] = vread(i + VPF);
          const int ks = i / C::DB, db = i % C::DB;
          oacc[db] = mfma32x32x16<BF16>(vfr[i], pf[ks], oacc[db]);
        }
        __builtin_amdgcn_sched_group_barrier(kSchedValu, 8, 0);
#pragma unroll
        for (int i = NPVB; i < NPV - VPF; ++i) {
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, VPF, 0);
        if constexpr (D >= 128) __builtin_amdgcn_s_setprio(0);
        return;
      }
      // Written in issue order (read i + KPF, MFMA i, DMA i), which also
      // bounds the fragments' live ranges if the schedule below is relaxed.
      auto kread = [&](int i) {
        const int s = i / (BN / 32), kb = i % (BN / 32);
        return *(const u32x4_t *)(sbase + kro[s] + 32 * kb * C::ROW);
      };
#pragma unroll
      for (int i = 0; i < KPF && i < NQK; ++i) kfr[i] = kread(i);
      static_assert(NDMA <= NQK, "one DMA per QK MFMA at most");
#pragma unroll
      for (int i = 0; i < NQK; ++i) {
        if (i + KPF < NQK) kfr[i + KPF] = kread(i + KPF);
        if (i + KPF == NQK) {
#pragma unroll
          for (int j = 0; j < VPF; ++j) {
            if constexpr (V8)
              vfr8[j] = vread8(j);
            else
              vfr[j] = vread(j);
          }
        }
        const int s = i / (BN / 32), kb = i % (BN / 32);
        sacc[kb] = mfma32x32x16<BF16>(kfr[i], qf[s], sacc[kb]);
        if (i < NDMA) dma(NEXT{}, rk_n, rv_n, i);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, KPF, 0);
#pragma unroll
      for (int i = 0; i < NQK; ++i) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        if (i < NDMA) __builtin_amdgcn_sched_group_barrier(kSchedVmem, 1, 0);
        if (i + KPF < NQK) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
        if (i + KPF == NQK) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, VRD * VPF, 0);
      }

      if (MASKED) {
#pragma unroll
        for (int kb = 0; kb < BN / 32; ++kb) mask_block(kb);
      }

      // Row max of the tile in log2 units (both lane halves of a row).
      auto tile_max = [&]() __attribute__((always_inline)) {
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kb][r]);
        return halves_max(mx) * c;
      };
      // p = 2^(s c - mb) into pacc, and this lane's sum of them (half a row).
      float part = 0.f;
      auto exps = [&](float m) __attribute__((always_inline)) {
        const float mb = (m == -INFINITY) ? 0.f : m;
        float lsum[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float pv = fast_exp2(__builtin_fmaf(sacc[kb][r], c, -mb));
            pacc[kb][r] = pv;
            lsum[r & 3] = (kb == 0 && r < 4) ? pv : lsum[r & 3] + pv;
          }
        part = (lsum[0] + lsum[1]) + (lsum[2] + lsum[3]);
      };
      if constexpr (kSumTrigger && EXACT) {
        // A unit's first tile: every running max is still -inf and O = 0,
        // l = 0, so the tile's row max becomes the running max (rows with no
        // visible key keep -inf and get p = 0).
        m_run = tile_max();
        exps(m_run);
      } else if constexpr (kSumTrigger) {
        // Later tiles use the running max as it stands, so the row max costs
        // nothing on most tiles.  It moves only when a lane's sum of p over
        // the tile exceeds kLazyMaxSum (which bounds each p).  Then (rare: a
        // logit beyond any seen before by 14 or 32 log2 units) the tile's row max becomes
        // the running max, O and l are rescaled and p is recomputed from the
        // scores, which are kept.  Exact by shift invariance; NaN or inf
        // sums also take the exact path.
        exps(m_run);
        if (__builtin_amdgcn_ballot_w64(!(part <= kLazyMaxSum<BF16 && !V8>))) {
          const float m_new = fmaxf(m_run, tile_max());
          rescale(m_new == m_run ? 1.f : fast_exp2(m_run - m_new));
          m_run = m_new;
          exps(m_run);
        }
      } else {
        // The row max of every tile, moved lazily (by more than 2^8 only).
        // Rows whose running max is still -inf hold O = 0 and l = 0: nothing
        // to rescale (every row in a unit's first tile), except in the D = 128
        // kernels at three workgroups per CU, whose 168-register budget the
        // extra compare overflows (a spill); alpha = 0 keeps such rows at 0.
        constexpr bool kSkipFirstRescale = !(D >= 128 && OCC >= 3);
        const float m_cand = tile_max();
        const bool upd = m_cand > m_run + kLazyMaxThreshold;
        const float m_new = upd ? m_cand : m_run;
        if (__builtin_amdgcn_ballot_w64(upd && (!kSkipFirstRescale || m_run != -INFINITY)))
          rescale(upd ? fast_exp2(m_run - m_new) : 1.f);
        m_run = m_new;
        exps(m_run);
      }

      if constexpr (V8) {
        // P^T in e5m2 (round to nearest even), per 64-key chunk kc: byte j =
        // register j % 16 of block 2kc + j / 16, four bytes per VGPR.
        i32x8_t pf8[BN / 64];
#pragma unroll
        for (int kc = 0; kc < BN / 64; ++kc)
#pragma unroll
          for (int w = 0; w < 8; ++w) {
            const int kb = 2 * kc + (w >> 2), r0 = 4 * (w & 3);
            const int lo = __builtin_amdgcn_cvt_pk_bf8_f32(pacc[kb][r0], pacc[kb][r0 + 1], 0, false);
            pf8[kc][w] = __builtin_amdgcn_cvt_pk_bf8_f32(pacc[kb][r0 + 2], pacc[kb][r0 + 3], lo, true);
          }
        l_run += part;
        // O^T += V^T P^T: one fp8 MFMA per (64 keys, 32 head dims) (unit
        // scales: E8M0 exponent 127 = 2^0), the next fragment's four reads
        // ahead of it.
#pragma unroll
        for (int i = 0; i < NPV; ++i) {
          if (i + VPF < NPV) vfr8[i + VPF] = vread8(i + VPF);
          const int kc = i / C::DB, db = i % C::DB;
          oacc[db] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(vfr8[i], pf8[kc], oacc[db], 1, 1, 0, 127, 0, 127);
        }
#pragma unroll
        for (int i = 0; i < NPV - VPF; ++i) {
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedDsRead, VRD, 0);
        }
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, VPF, 0);
      } else {
      // P^T fragments: k-step ks (16 keys) = registers 8t..8t+7 of block ks/2.
      u32x4_t pf[BN / 16];
#pragma unroll
      for (int ks = 0; ks < BN / 16; ++ks) {
        const int kb = ks >> 1, t8 = (ks & 1) * 8;
#pragma unroll
        for (int w = 0; w < 4; ++w) pf[ks][w] = pack2<BF16>(pacc[kb][t8 + 2 * w], pacc[kb][t8 + 2 * w + 1]);
      }
      if constexpr (!MSUM) l_run += part;

      // O^T += V^T P^T; the A operand is two transpose reads (keys +0..3 and
      // +8..11 of the k-step), VPF fragments ahead of their MFMA.  For
      // D >= 128 the wave raises its issue priority over these MFMAs, so the
      // other wave of the SIMD does not hold them back with its softmax
      // (measured 1.5-2% on B4 H32 S2048 and B2 H16 S8192 causal; at D = 64
      // it cost 2-4%, and raising it over the QK MFMAs or the softmax did not
      // pay).
      if constexpr (D >= 128) __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int i = 0; i < NPV; ++i) {
        if (i + VPF < NPV) vfr[i + VPF] = vread(i + VPF);
        const int ks = i / C::DB, db = i % C::DB;
        oacc[db] = mfma32x32x16<BF16>(vfr[i], pf[ks], oacc[db]);
      }
      if constexpr (MSUM) {
#pragma unroll
        for (int ks = 0; ks < BN / 16; ++ks) lacc = mfma32x32x16<BF16>(ones, pf[ks], lacc);
      }
#pragma unroll
      for (int i = 0; i < NPV - VPF; ++i) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, VPF + (MSUM ? BN / 16 : 0), 0);
      if constexpr (D >= 128) __builtin_amdgcn_s_setprio(0);
      }
    };

    // Tiles visible to every query of the workgroup need no mask.  Each run
    // of tiles steps t in stage pairs (t even -> stage 0).
    const int n_full = n_full_of(q0);
    using NotFirst = std::integral_constant<bool, false>;
    using Whole = std::integral_constant<bool, false>;
    int t = t_begin;
    auto run = [&](int end, auto masked_tag) __attribute__((always_inline)) {
      if (t < end && (t & 1)) kv_tile(t++, masked_tag, S1{}, NotFirst{}, Whole{});
      for (; t + 1 < end; t += 2) {
        kv_tile(t, masked_tag, S0{}, NotFirst{}, Whole{});
        kv_tile(t + 1, masked_tag, S1{}, NotFirst{}, Whole{});
      }
      if (t < end) kv_tile(t++, masked_tag, S0{}, NotFirst{}, Whole{});
    };
    // The unit's first tile (it sets the running max), in its stage.
    auto first_tile = [&](auto masked_tag) __attribute__((always_inline)) {
      using First = std::integral_constant<bool, true>;
      if (t & 1)
        kv_tile(t, masked_tag, S1{}, First{}, Whole{});
      else
        kv_tile(t, masked_tag, S0{}, First{}, Whole{});
      ++t;
    };
    // Tiles [t, end) in which this wave has nothing to compute: only keep the
    // DMA ring and the barriers in step with the other waves (one barrier
    // per tile, like kv_tile).
    auto idle_tiles = [&](int end) __attribute__((always_inline)) {
      for (; t < end; ++t) {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        __syncthreads();
        BufRsrc rk_n, rv_n;
        tile_rsrc(t + 1, &rk_n, &rv_n);
        if (late_ticket && t == t_last && threadIdx.x == 0) next_raw = tq.request();
        if (t & 1) {
#pragma unroll
          for (int i = 0; i < C::NDMA; ++i) dma(S0{}, rk_n, rv_n, i);
        } else {
#pragma unroll
          for (int i = 0; i < C::NDMA; ++i) dma(S1{}, rk_n, rv_n, i);
        }
#ifdef FA_TIMING
        tm_idle += 1;
#endif
      }
    };
    // When another workgroup's wave shares the SIMD (OCC >= 2), a wave skips
    // the tiles it has no work in: all of them when none of its rows is in
    // range (the ragged last m-tile; its stores then fall past the buffers'
    // ranges and are dropped), and under the causal mask the tiles past its
    // last row (visibility is monotone in t).  Skipping at this level, not
    // inside the tile body, keeps the tile code's register allocation: an
    // early return there cost the causal kernels 54 registers.  With one
    // workgroup per CU every wave computes every tile (fully masked tiles
    // give p = 0): the workgroup waits for its last wave either way.
    if (OCC >= 2 && q0w >= p.Sq) {
      idle_tiles(n_tiles);
    } else {
      using Unmasked = std::integral_constant<bool, false>;
      using Masked = std::integral_constant<bool, true>;
      const int n_act = (CAUSAL && OCC >= 2) ? max(n_full, min(n_tiles, wave_last_q / BN + 1)) : n_tiles;
      if constexpr (kSumTrigger) {
        if (t < n_full)
          first_tile(Unmasked{});
        else if (t < n_act)
          first_tile(Masked{});
      }
      // Causal: when the wave's rows end in the first 32 keys of its last
      // tile (and that tile is masked and not the unit's first), the second
      // block is masked for all of them and the tile runs as a half tile.
      constexpr bool kHalfTiles = CAUSAL && OCC >= 2 && kSumTrigger && !V8 && BN == 64;
      const bool half_last =
          kHalfTiles && n_act - 1 > max(n_full - 1, t_begin) && wave_last_q - (n_act - 1) * BN < 32;
      run(n_full, Unmasked{});
      run(half_last ? n_act - 1 : n_act, Masked{});
      if constexpr (kHalfTiles) {
        if (half_last) {
          using Half = std::integral_constant<bool, true>;
          if (t & 1)
            kv_tile(t, Masked{}, S1{}, NotFirst{}, Half{});
          else
            kv_tile(t, Masked{}, S0{}, NotFirst{}, Half{});
          ++t;
        }
      }
      idle_tiles(n_tiles);
    }
#ifdef FA_TIMING
    tm_epi0 = FA_CLK() - tm0;
#endif

    // The DMAs issued during the last KV tile (zeros into the free stage)
    // must land before the next unit's DMAs target that stage.  Wait for
    // them here, before the output stores: vmcnt retires in issue order, so
    // a wait after the stores would also wait for their write acknowledgement
    // (a memory round trip per unit), which the next unit's first wait now
    // overlaps with its own loads.
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    const float l_tot = MSUM ? lacc[0] : halves_sum(l_run);
    if (p.kv_splits > 1) {
      // Partial result of this KV run: O normalised by its own row sum, in
      // fp32, and its natural-log LSE (-inf, with O = 0, where no key of the
      // run is visible to the row).
      const float inv_p = l_tot > 0.f ? 1.f / l_tot : 0.f;
      const int64_t unit = (int64_t)split * p.B * p.H + bh;
      const BufRsrc rpo = make_rsrc(p.part_o + unit * p.Sq * D, (uint32_t)((int64_t)p.Sq * D * 4));
      const uint32_t po = (uint32_t)(qrow * D * 4 + 16 * h);
#pragma unroll
      for (int db = 0; db < C::DB; ++db)
#pragma unroll
        for (int j = 0; j < (D >= 32 ? 4 : 2); ++j) {
          u32x4_t x;
#pragma unroll
          for (int i = 0; i < 4; ++i) x[i] = __builtin_bit_cast(uint32_t, oacc[db][4 * j + i] * inv_p);
          buf_store16(x, rpo, po + 4 * (32 * db + 8 * j));
        }
      const uint32_t nbytes = (uint32_t)p.Sq * 4u;
      const BufRsrc rpl = make_rsrc(p.part_lse + unit * p.Sq, nbytes);
      const float lse = l_tot > 0.f ? (m_run + __log2f(l_tot)) * kLn2 : -INFINITY;
      buf_store4(__builtin_bit_cast(uint32_t, lse), rpl, h ? nbytes : (uint32_t)qrow * 4u);
    } else {
    const float inv = 1.f / l_tot;
    const char *og = p.o + 2 * (bb * p.o_sb + hh * p.o_sh);
    const BufRsrc ro = make_rsrc(og, (uint32_t)((int64_t)p.Sq * p.o_ss * 2));
    // A lane holds 4-dim pieces of one row of O (the O^T layout), so storing
    // them directly makes every store instruction touch 32 rows.  Staged
    // stores send O through LDS instead, and each instruction writes whole
    // rows: the wave writes its 32 rows into the 1 KB LDS chunks that only
    // its own DMAs fill, in the stage that received the last tile's (empty)
    // DMAs.  Those have landed (vmcnt above), no other wave reads that stage
    // after the last tile's barrier, and the next unit's DMAs wait for the
    // barrier at the end of this unit.  It then reads them back one chunk per
    // instruction and stores 16 bytes per lane along the rows.  Kernels whose
    // DMAs fill fewer chunks than 32 rows take (32-key tiles, 64-key fp8 V)
    // run two passes over the halves of the head dims; 16-byte units of a row
    // are XOR-swizzled by the row, so the 32 rows of a write spread over the
    // banks.  The D = 128 kernels at three workgroups per CU keep the direct
    // stores: their 168-register budget has no room for the staging (2
    // registers spilled).
    constexpr bool kStagedStore = !(D >= 128 && OCC >= 3);
    if constexpr (kStagedStore) {
      constexpr int kOwn = C::NDMA;          // 1 KB chunks this wave's DMAs fill
      constexpr int kNeed = D / 16;          // KB of 32 rows of 2 D bytes
      constexpr int NPASS = kOwn >= kNeed ? 1 : 2;
      static_assert(NPASS * kOwn >= kNeed && (NPASS == 1 || C::DB % 2 == 0), "O staging space");
      constexpr int W = 2 * D / NPASS;       // bytes of a row per pass
      constexpr int RPC = 1024 / W;          // rows per chunk
      constexpr int U = W / 16;              // 16-byte units per row segment
      constexpr int USW = U < 32 ? U : 32;   // swizzle span
      constexpr int DBP = C::DB / NPASS;
      constexpr int JN = D >= 32 ? 4 : 2;
      constexpr int NR = 32 / RPC;           // chunks per pass
      constexpr int RG = NR < 4 ? NR : 4;    // chunks read per group
      char *const fs = (n_tiles & 1) ? smem1 : smem0;
      // Lane and wave indices made opaque here, so that the addresses below
      // (which depend on nothing else) are not hoisted out of the unit loop
      // and kept live through every tile.
      int ln = lane, wv = wave;
      asm volatile("" : "+v"(ln), "+s"(wv));
      const int ln_n = ln & 31, ln_h = ln >> 5;
      auto own = [&](int k) __attribute__((always_inline)) {
        return k < C::IPW ? (uint32_t)((wv + k * NW) * 1024)
                          : (uint32_t)(C::TILE + (wv + (k - C::IPW) * NW) * 1024);
      };
      const uint32_t wbase = own(ln_n / RPC) + (uint32_t)((ln_n % RPC) * W + 8 * ln_h);
      const int wsw = ln_n & (USW - 1);
      const int rr = ln / U, lu = ln % U;
      // Scheduling barriers keep the writes of one block, and the reads of
      // four chunks, apart from the next ones: hoisted together they would
      // hold every packed row or read chunk in registers at once.
#pragma unroll
      for (int ps = 0; ps < NPASS; ++ps) {
#pragma unroll
        for (int db = ps * DBP; db < (ps + 1) * DBP; ++db) {
#pragma unroll
          for (int j = 0; j < JN; ++j) {  // dims 32db + 8j + 4h + 0..3: unit 4 (db - ps DBP) + j, half h
            u32x2_t x;
            x[0] = pack2<BF16>(oacc[db][4 * j + 0] * inv, oacc[db][4 * j + 1] * inv);
            x[1] = pack2<BF16>(oacc[db][4 * j + 2] * inv, oacc[db][4 * j + 3] * inv);
            const int u = 4 * (db - ps * DBP) + j;
            *(u32x2_t *)(fs + wbase + ((u ^ wsw) << 4)) = x;
          }
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int r0 = 0; r0 < NR; r0 += RG) {
          u32x4_t x[RG];
#pragma unroll
          for (int i = 0; i < RG; ++i) {
            const int row = (r0 + i) * RPC + rr;
            x[i] = *(const u32x4_t *)(fs + own(r0 + i) + rr * W + ((lu ^ (row & (USW - 1))) << 4));
          }
#pragma unroll
          for (int i = 0; i < RG; ++i)
            buf_store16(x[i], ro, (uint32_t)((q0w + (r0 + i) * RPC + rr) * p.o_ss * 2 + ps * W + lu * 16));
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    } else {
      const uint32_t oo = (uint32_t)(qrow * p.o_ss * 2 + 8 * h);
#pragma unroll
      for (int db = 0; db < C::DB; ++db)
#pragma unroll
        for (int j = 0; j < (D >= 32 ? 4 : 2); ++j) {  // rows 8j + 4h + 0..3 of the block
          u32x2_t x;
          x[0] = pack2<BF16>(oacc[db][4 * j + 0] * inv, oacc[db][4 * j + 1] * inv);
          x[1] = pack2<BF16>(oacc[db][4 * j + 2] * inv, oacc[db][4 * j + 3] * inv);
          buf_store8(x, ro, oo + 2 * (32 * db + 8 * j));
        }
    }
    if (p.lse != nullptr) {
      const uint32_t nbytes = (uint32_t)p.Sq * 4u;
      const BufRsrc rl = make_rsrc(p.lse + ((int64_t)bb * p.H + hh) * p.Sq, nbytes);
      const float lse = (m_run + __log2f(l_tot)) * kLn2;
      buf_store4(__builtin_bit_cast(uint32_t, lse), rl, h ? nbytes : (uint32_t)qrow * 4u);
    }
    }
#ifdef FA_TIMING
    if (p.timing != nullptr && lane == 0) {
      uint32_t *dst = p.timing + ((int64_t)(mt * p.B * p.H + bh) * NW + wave) * 16;
      dst[0] = tm_vm; dst[1] = tm_bar; dst[2] = tm_cmp; dst[3] = n_comp;
      dst[4] = tm_pro; dst[5] = FA_CLK() - tm0; dst[6] = n_tiles; dst[7] = tm_epi0;
      dst[8] = rt0; dst[9] = (uint32_t)__builtin_amdgcn_s_memrealtime();
      dst[10] = __builtin_amdgcn_s_getreg(4 | (0 << 6) | (31 << 11));   // HW_ID
      dst[11] = __builtin_amdgcn_s_getreg(20 | (0 << 6) | (31 << 11));  // XCC_ID
      dst[12] = blockIdx.x + (it << 16);
      dst[13] = tm_dma; dst[14] = tm_idle;
    }
#endif
    if (threadIdx.x == 0) s_ticket[(it + 1) & 1] = tq.finish(next_raw, it);
    __syncthreads();  // LDS reuse by the next tile, ticket broadcast
  }
}

// ---------------------------------------------------------------------------
// Ping-pong kernel: 8 waves in two groups of 4.  Waves w and w + 4
// share a SIMD.  Every wave runs the same action list
//     M(0) S(0) M(1) S(1) ... M(n)
// with  M(t) = O^T += V^T(t-1) P^T(t-1) and S^T(t) = K(t) Q^T  (32 MFMAs) and
//       S(t) = online softmax of S^T(t) -> P(t), rescale O  (VALU),
// one action per barrier interval, group 1 one interval behind group 0: in
// every interval one wave of each SIMD issues MFMAs while the other runs the
// softmax, so the matrix core is fed while the exp/max/sum work proceeds.
// K and V tiles come in by DMA into two LDS rings of NR slots each.  K(t) is
// read in intervals 2t, 2t+1 and V(t) in 2t+2, 2t+3; at the start of
// interval 2j the DMAs for K(j + NR - 1) and V(j + NR - 2) are issued into
// the slots freed by K(j - 1) and V(j - 2), so every tile has 2 NR - 2
// intervals to arrive.  Past the last tile the same DMAs are issued against an
// empty buffer range (they write zeros into free slots), which keeps the
// number in flight, and so the vmcnt allowance, uniform.
template <int D, int BN, int NR>
struct Cfg3 {
  static constexpr int NW = 8;
  static constexpr int BM = 32 * NW;
  static constexpr int ROW = 2 * D;
  static constexpr int CPR = ROW / 16;
  static constexpr int RPI = 1024 / ROW;
  static constexpr int TILE = BN * ROW;
  static constexpr int IPT = TILE / 1024;
  static constexpr int IPW = IPT / NW;
  static constexpr int K_OFF = 0;
  static constexpr int V_OFF = NR * TILE;
  static constexpr int LDS_BYTES = 2 * NR * TILE;
  static_assert(CPR >= 8 && IPT % NW == 0 && IPW >= 1, "tile shape");
  static_assert(NR >= 3 && NR <= 6, "ring depth");
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget of one gfx950 CU");
};

template <int D, int BN, int NR, bool BF16, bool CAUSAL>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
fa_fwd_pp_kernel(KernelArgs p) {
  using C = Cfg3<D, BN, NR>;
  constexpr int NW = C::NW;
  constexpr int BM = C::BM;
  __shared__ __attribute__((aligned(1024))) char smem[C::LDS_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;
  // 32-row blocks alternate between the groups, so diagonal tiles cost both
  // groups about the same.
  const int rblk = 2 * (wave & 3) + grp;
  const int n = lane & 31;
  const int h = lane >> 5;

  uint32_t dk[C::IPW], dv[C::IPW];
#pragma unroll
  for (int j = 0; j < C::IPW; ++j) {
    const int row = (wave + j * NW) * C::RPI + lane / C::CPR;
    const int lc = (lane % C::CPR) ^ swz<D>(row);
    dk[j] = (uint32_t)(row * p.k_ss * 2 + lc * 16);
    dv[j] = (uint32_t)(row * p.v_ss * 2 + lc * 16);
  }
  uint32_t kro[D / 16];
#pragma unroll
  for (int s = 0; s < D / 16; ++s) kro[s] = (uint32_t)(n * C::ROW + (((2 * s + h) ^ swz<D>(n)) * 16));
  uint32_t vro[D / 32][2];
  {
    const int g = lane >> 4, sg = lane & 15, jj = sg >> 2, cc = sg & 3;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int row = 8 * e + 4 * h + jj;
        const int lc = 4 * db + 2 * (g & 1) + (cc >> 1);
        vro[db][e] = (uint32_t)((4 * h + jj) * C::ROW + ((lc ^ swz<D>(row)) * 16) + (cc & 1) * 8);
      }
  }

  const float c = p.c;
  const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_char *)smem;

  // Tile loop: thread 0 takes tickets (the next one is requested at the top
  // of a tile and published through LDS at its end, behind a barrier).
  __shared__ uint32_t s_ticket[2];
  const TileQueue tq(p);
  int bh, mt, split;
  for (int it = 0; tq.tile(it == 0 ? tq.first() : s_ticket[it & 1], p.n_mtiles, CAUSAL, p.q_group, p.q_bands,
                           &bh, &mt, &split);
       ++it) {
    unsigned long long next_raw = 0;
    if (threadIdx.x == 0) next_raw = tq.request();
#ifdef FA_TIMING
    uint32_t tm_m = 0, tm_s = 0, tm_w = 0, tm_dma = 0, tm_pro = 0, tm_epi = 0, n_m = 0, n_s = 0;
    const uint32_t tm0 = FA_CLK();
    uint32_t tmark = tm0;
#endif
    const int bb = bh / p.H;
    const int hh = bh - bb * p.H;

    const int q0 = mt * BM;
    const int q0w = q0 + 32 * rblk;
    const int qrow = q0w + n;

    const char *qg = p.q + 2 * (bb * p.q_sb + hh * p.q_sh);
    const char *kg = p.k + 2 * (bb * p.k_sb + hh * p.k_sh);
    const char *vg = p.v + 2 * (bb * p.v_sb + hh * p.v_sh);

    const int kv_end = CAUSAL ? min(p.Sk, q0 + BM) : p.Sk;
    const int n_tiles = (kv_end + BN - 1) / BN;
    const int wave_last_q = q0w + 31;
    // Tiles [0, n_full) are visible to every row of this wave (no mask);
    // tile t is active for this wave iff some key of it is visible.
    int n_full = p.Sk / BN;
    if (CAUSAL) n_full = min(n_full, (q0w + 1) / BN);
    n_full = min(n_full, n_tiles);
    auto active = [&](int t) { return !CAUSAL || t * BN <= wave_last_q; };

    // DMA of K(t) / V(t) into ring slot t % NR.  One descriptor per (b, h)
    // spans keys [0, Sk); the tile offset rides in the lane offset, so rows
    // at or past Sk (ragged tail, tiles past the end) read as zeros.
    const BufRsrc rk = make_rsrc(kg, (uint32_t)((int64_t)p.Sk * p.k_ss * 2));
    const BufRsrc rv = make_rsrc(vg, (uint32_t)((int64_t)p.Sk * p.v_ss * 2));
    const uint32_t k_tile_bytes = (uint32_t)(BN * p.k_ss * 2);
    const uint32_t v_tile_bytes = (uint32_t)(BN * p.v_ss * 2);
    auto issue_k = [&](int t) {
      const uint32_t st = lds_base + (uint32_t)(C::K_OFF + (t % NR) * C::TILE);
      const uint32_t off = (uint32_t)t * k_tile_bytes;
#pragma unroll
      for (int j = 0; j < C::IPW; ++j) dma16(rk, st + (uint32_t)((wave + j * NW) * 1024), dk[j] + off);
    };
    auto issue_v = [&](int t) {
      const uint32_t st = lds_base + (uint32_t)(C::V_OFF + (t % NR) * C::TILE);
      const uint32_t off = (uint32_t)t * v_tile_bytes;
#pragma unroll
      for (int j = 0; j < C::IPW; ++j) dma16(rv, st + (uint32_t)((wave + j * NW) * 1024), dv[j] + off);
    };

    u32x4_t qf[D / 16];
    {
      const BufRsrc rq = make_rsrc(qg, (uint32_t)((int64_t)p.Sq * p.q_ss * 2));
      const uint32_t qo = (uint32_t)(qrow * p.q_ss * 2 + 16 * h);
#pragma unroll
      for (int s = 0; s < D / 16; ++s) qf[s] = buf_load16(rq, qo + 32 * s) ^ p.q_sign;
    }
    // Prologue: K(0 .. NR-2) and V(0 .. NR-3); Q and these have landed
    // (this wave's), then everyone's.
    issue_k(0);
#pragma unroll
    for (int i = -(NR - 2); i < 0; ++i) {
      issue_k(i + NR - 1);
      if (i + NR - 2 >= 0) issue_v(i + NR - 2);
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();
#ifdef FA_TIMING
    { const uint32_t now = FA_CLK(); tm_pro += FA_CLK_DELTA(tmark, now); tmark = now; }
#endif

    f32x16_t oacc[D / 32];
#pragma unroll
    for (int db = 0; db < D / 32; ++db) oacc[db] = (f32x16_t){};
    float m_run = -INFINITY;
    float l_run = 0.f;
    f32x16_t sacc[BN / 32];
    u32x4_t pf[BN / 16];

    // Interval k starts (after the previous barrier) by issuing, when k = 2j,
    // the DMAs for K(j + NR - 1) and V(j + NR - 2), and ends with a barrier.
    // Before the barrier that opens interval 2j this wave's DMAs of K(j) and
    // V(j - 1) have landed: only the groups issued in the last min(NR - 2, j)
    // even intervals may still be in flight.
    int k = 0;
#ifdef FA_TIMING
    uint32_t tphase = 0;
#define FA_TAG_M() (tm_m += tphase, ++n_m)
#define FA_TAG_S() (tm_s += tphase, ++n_s)
#else
#define FA_TAG_M() ((void)0)
#define FA_TAG_S() ((void)0)
#endif
    auto interval_start = [&]() {
#ifdef FA_TIMING
      tmark = FA_CLK();
#endif
      if ((k & 1) == 0) {
        const int j = k >> 1;
        issue_k(j + NR - 1);
        issue_v(j + NR - 2);
      }
    };
    auto interval_end = [&]() {
#ifdef FA_TIMING
      const uint32_t tend = FA_CLK();
#endif
      if (k & 1) {
        const int j = (k + 1) >> 1;
        constexpr int G = 2 * C::IPW;  // DMA instructions per group
        if (j >= NR - 2) {
          __builtin_amdgcn_s_waitcnt(vmcnt_imm((NR - 2) * G));
        } else if (j == 1) {
          __builtin_amdgcn_s_waitcnt(vmcnt_imm(G));
        } else if (j == 2) {
          __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * G));
        } else {
          __builtin_amdgcn_s_waitcnt(vmcnt_imm(3 * G));
        }
      }
#ifdef FA_TIMING
      const uint32_t tdma = FA_CLK();
      tm_dma += FA_CLK_DELTA(tend, tdma);
#endif
      __syncthreads();
      ++k;
#ifdef FA_TIMING
      tm_w += FA_CLK_DELTA(tdma, FA_CLK());
      tphase = FA_CLK_DELTA(tmark, tend);
#endif
    };

    // M(t): PV(t-1) then QK(t), operand reads MPF MFMAs ahead.  The wave
    // raises its issue priority for the phase, so the other group's softmax
    // fills the gaps between its MFMAs instead of delaying them (4-5% on
    // B4 H32 S2048, B2 H16 S8192 and B8 H32 S3000 causal).
    auto mphase = [&](int t, auto pv_tag, auto qk_tag) {
      __builtin_amdgcn_s_setprio(1);
      constexpr bool DO_PV = decltype(pv_tag)::value;
      constexpr bool DO_QK = decltype(qk_tag)::value;
      constexpr int NPV = DO_PV ? (BN / 16) * (D / 32) : 0;
      constexpr int NQK = DO_QK ? (D / 16) * (BN / 32) : 0;
      constexpr int NOPS = NPV + NQK;
      constexpr int MPF = 3;
      const uint32_t stv = (uint32_t)(C::V_OFF + ((t + NR - 1) % NR) * C::TILE);
      const uint32_t stk = (uint32_t)(C::K_OFF + (t % NR) * C::TILE);
      u32x4_t fr[NOPS > 0 ? NOPS : 1];
#pragma unroll
      for (int i = 0; i < NOPS; ++i) {
        if (i < NPV) {
          const int ks = i / (D / 32), db = i % (D / 32);
          const uint32_t imm = stv + (uint32_t)(16 * ks * C::ROW);
          const u32x2_t lo = lds_read_tr16(smem, vro[db][0] + imm);
          const u32x2_t hi = lds_read_tr16(smem, vro[db][1] + imm + 8 * C::ROW);
          fr[i] = (u32x4_t){lo[0], lo[1], hi[0], hi[1]};
        } else {
          const int j = i - NPV;
          const int s = j / (BN / 32), kb = j % (BN / 32);
          fr[i] = *(const u32x4_t *)(smem + stk + kro[s] + 32 * kb * C::ROW);
        }
      }
      if constexpr (DO_QK) {
#pragma unroll
        for (int kb = 0; kb < BN / 32; ++kb) sacc[kb] = (f32x16_t){};
      }
#pragma unroll
      for (int i = 0; i < NOPS; ++i) {
        if (i < NPV) {
          const int ks = i / (D / 32), db = i % (D / 32);
          oacc[db] = mfma32x32x16<BF16>(fr[i], pf[ks], oacc[db]);
        } else {
          const int j = i - NPV;
          const int s = j / (BN / 32), kb = j % (BN / 32);
          sacc[kb] = mfma32x32x16<BF16>(fr[i], qf[s], sacc[kb]);
        }
      }
      // Pin the order: reads of the first MPF ops, then one MFMA and the
      // reads of the op MPF ahead, and so on.
#pragma unroll
      for (int i = 0; i < (MPF < NOPS ? MPF : NOPS); ++i) {
        if (i < NPV) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
        else __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
      }
#pragma unroll
      for (int i = 0; i + MPF < NOPS; ++i) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        if (i + MPF < NPV) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
        else __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, MPF < NOPS ? MPF : NOPS, 0);
      __builtin_amdgcn_s_setprio(0);
    };

    // S(t): mask (diagonal / ragged tail only), online softmax, rescale O, P(t).
    auto sphase = [&](int t, auto masked_tag) {
      constexpr bool MASKED = decltype(masked_tag)::value;
      const int kbase = t * BN;
      if (MASKED) {
        const int last_key = CAUSAL ? min(qrow, p.Sk - 1) : p.Sk - 1;
        const int lim = last_key - kbase - 4 * h;
#pragma unroll
        for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int off = 32 * kb + 8 * (r >> 2) + (r & 3);
            sacc[kb][r] = off <= lim ? sacc[kb][r] : -INFINITY;
          }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kb][r]);
      mx = halves_max(mx);
      const float m_cand = mx * c;
      const bool upd = m_cand > m_run + kLazyMaxThreshold;
      const float m_new = upd ? m_cand : m_run;
      // Rows whose running max is still -inf have O = 0 and l = 0: nothing to rescale
      // (every row in a unit's first tile).
      if (__builtin_amdgcn_ballot_w64(upd && m_run != -INFINITY)) {
        const float alpha = upd ? fast_exp2(m_run - m_new) : 1.f;
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < D / 32; ++db) oacc[db] *= alpha;
      }
      m_run = m_new;
      const float mb = (m_new == -INFINITY) ? 0.f : m_new;
      float lsum[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float pv = fast_exp2(__builtin_fmaf(sacc[kb][r], c, -mb));
          sacc[kb][r] = pv;
          lsum[r & 3] += pv;
        }
      l_run += (lsum[0] + lsum[1]) + (lsum[2] + lsum[3]);
#pragma unroll
      for (int ks = 0; ks < BN / 16; ++ks) {
        const int kb = ks >> 1, t8 = (ks & 1) * 8;
#pragma unroll
        for (int w = 0; w < 4; ++w) pf[ks][w] = pack2<BF16>(sacc[kb][t8 + 2 * w], sacc[kb][t8 + 2 * w + 1]);
      }
    };

    // Action list of this wave: M(0) S(0) ... M(n_act-1) S(n_act-1) M(n_act),
    // M(n_act) being P*V only, then idle intervals up to 2 n_tiles + 1
    // actions (tiles beyond n_act are above this wave's rows).  Visibility is
    // monotone in t, so the loops below need no per-tile branching.
    using T_ = std::integral_constant<bool, true>;
    using F_ = std::integral_constant<bool, false>;
    int n_act = n_tiles;
    if (CAUSAL) n_act = min(n_act, wave_last_q / BN + 1);
    if (grp == 1) {  // group 1 starts one interval late
      interval_start();
      interval_end();
    }
    // t = 0 (n_act >= 1 always): QK only.
    interval_start();
    mphase(0, F_{}, T_{});
    interval_end();
    FA_TAG_M();
    interval_start();
    if (0 < n_full) sphase(0, F_{}); else sphase(0, T_{});
    interval_end();
    FA_TAG_S();
    int t = 1;
    for (; t < n_full; ++t) {
      interval_start();
      mphase(t, T_{}, T_{});
      interval_end();
      FA_TAG_M();
      interval_start();
      sphase(t, F_{});
      interval_end();
      FA_TAG_S();
    }
    for (; t < n_act; ++t) {
      interval_start();
      mphase(t, T_{}, T_{});
      interval_end();
      FA_TAG_M();
      interval_start();
      sphase(t, T_{});
      interval_end();
      FA_TAG_S();
    }
    interval_start();
    mphase(n_act, T_{}, F_{});
    interval_end();
    FA_TAG_M();
    for (int idle = 2 * (n_tiles - n_act); idle > 0; --idle) {
      interval_start();
      interval_end();
    }
    if (grp == 0) {  // group 0's last interval is idle
      interval_start();
      interval_end();
    }

    const float l_tot = halves_sum(l_run);
    const float inv = 1.f / l_tot;
    {
      const char *og = p.o + 2 * (bb * p.o_sb + hh * p.o_sh);
      const BufRsrc ro = make_rsrc(og, (uint32_t)((int64_t)p.Sq * p.o_ss * 2));
      const uint32_t oo = (uint32_t)(qrow * p.o_ss * 2 + 8 * h);
#pragma unroll
      for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          u32x2_t x;
          x[0] = pack2<BF16>(oacc[db][4 * j + 0] * inv, oacc[db][4 * j + 1] * inv);
          x[1] = pack2<BF16>(oacc[db][4 * j + 2] * inv, oacc[db][4 * j + 3] * inv);
          buf_store8(x, ro, oo + 2 * (32 * db + 8 * j));
        }
    }
    if (p.lse != nullptr) {
      const uint32_t nbytes = (uint32_t)p.Sq * 4u;
      const BufRsrc rl = make_rsrc(p.lse + ((int64_t)bb * p.H + hh) * p.Sq, nbytes);
      const float lse = (m_run + __log2f(l_tot)) * kLn2;
      buf_store4(__builtin_bit_cast(uint32_t, lse), rl, h ? nbytes : (uint32_t)qrow * 4u);
    }
#ifdef FA_TIMING
#undef FA_TAG_M
#undef FA_TAG_S
    if (p.timing != nullptr && lane == 0) {
      const uint32_t now = FA_CLK();
      tm_epi = FA_CLK_DELTA(tmark, now);
      uint32_t *dst = p.timing + ((int64_t)(mt * p.B * p.H + bh) * 8 + wave) * 8;
      dst[0] = tm_m; dst[1] = tm_s; dst[2] = tm_w; dst[3] = tm_pro; dst[4] = tm_dma;
      dst[5] = FA_CLK_DELTA(tm0, now); dst[6] = n_m; dst[7] = n_s;
    }
#endif
    // The DMAs issued past the last tile may still be writing zeros into the
    // rings: retire them (every wave) before a next tile reuses the slots.
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    if (threadIdx.x == 0) s_ticket[(it + 1) & 1] = tq.finish(next_raw, it);
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Split-KV merge.  With m = max_s LSE_s and w_s = exp(LSE_s - m),
//     LSE = m + ln(sum_s w_s),   O = sum_s w_s O_s / sum_s w_s,
// exact for partial results normalised by their own row sums (O_s) with
// natural-log LSE_s; runs with no visible key have LSE_s = -inf, w_s = 0.
// HBM-bound: reads splits * (D + 1) fp32 per row, writes D halves + 1 fp32.
// D / 4 lanes share a row, each loading 16 bytes of every O_s and storing
// 8 bytes of O, so a wave moves whole 64-byte segments (256 / D rows per
// wave, 1024 / D per block).
struct MergeArgs {
  const float *part_o;   // [splits][B*H][Sq][D]
  const float *part_lse; // [splits][B*H][Sq]
  char *o;
  float *lse;            // may be null
  int64_t o_sb, o_sh, o_ss;
  int32_t B, H, Sq, D, splits;
};

template <bool BF16>
__global__ void __launch_bounds__(256) fa_merge_kernel(MergeArgs a) {
  const int lpr_log2 = 29 - __builtin_clz((unsigned)a.D);  // log2(D / 4): D is a power of two
  const int li = threadIdx.x & ((1 << lpr_log2) - 1);       // this lane's 4 columns: 4 li .. 4 li + 3
  const int64_t rows = (int64_t)a.B * a.H * a.Sq;
  const int64_t row = ((int64_t)blockIdx.x << (8 - lpr_log2)) + (threadIdx.x >> lpr_log2);
  if (row >= rows) return;
  const int bh = (int)(row / a.Sq);
  const int q = (int)(row - (int64_t)bh * a.Sq);
  const int64_t plane = rows;  // rows per split
  float m = -INFINITY;
  for (int s = 0; s < a.splits; ++s) m = fmaxf(m, a.part_lse[s * plane + row]);
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  float wsum = 0.f;
#pragma unroll 4
  for (int s = 0; s < a.splits; ++s) {
    const float ls = a.part_lse[s * plane + row];
    const float w = ls == -INFINITY ? 0.f : fast_exp2((ls - m) * kLog2e);
    wsum += w;
    const f32x4_t x = *(const f32x4_t *)(a.part_o + (s * plane + row) * a.D + 4 * li);
    acc += w * x;
  }
  const float inv = 1.f / wsum;
  const int bb = bh / a.H, hh = bh - bb * a.H;
  char *dst = a.o + 2 * (bb * a.o_sb + hh * a.o_sh + (int64_t)q * a.o_ss);
  u32x2_t v;
  v[0] = pack2<BF16>(acc[0] * inv, acc[1] * inv);
  v[1] = pack2<BF16>(acc[2] * inv, acc[3] * inv);
  *(u32x2_t *)(dst + 8 * li) = v;
  if (a.lse != nullptr && li == 0) a.lse[row] = m + __logf(wsum);
}

// ---------------------------------------------------------------------------
// Kernel table: kKernelFns[i] is the kernel that kKernelMeta[i] (fa_plan.cpp)
// describes, instantiated from that entry's parameters; the LDS bytes the
// planner reports are checked against each kernel's own layout.
typedef void (*KernelFn)(KernelArgs);

template <int I>
KernelFn kernel_fn() {
  constexpr KernelMeta m = kKernelMeta[I];
  constexpr bool bf16 = out_is_bf16(m.dtype), v8 = v_is_fp8(m.dtype), causal = m.causal != 0;
  if constexpr (m.kind == kPingPong) {
    static_assert(m.NW == Cfg3<m.D, m.BN, m.stages>::NW, "ping-pong workgroup size");
    static_assert(Cfg3<m.D, m.BN, m.stages>::LDS_BYTES == kernel_lds_bytes(m), "LDS bytes");
    return fa_fwd_pp_kernel<m.D, m.BN, m.stages, bf16, causal>;
  } else {
    static_assert(Cfg2<m.D, m.BN, m.NW, m.stages, m.wg_per_cu, v8>::LDS_BYTES == kernel_lds_bytes(m), "LDS bytes");
    return fa_fwd_dma_kernel<m.D, m.BN, m.NW, m.stages, m.wg_per_cu, bf16, causal, v8>;
  }
}

template <int... I>
struct KernelFnTable {
  const KernelFn fns[sizeof...(I)] = {kernel_fn<I>()...};
};
template <int... I>
KernelFnTable<I...> make_kernel_fn_table(std::integer_sequence<int, I...>);
const decltype(make_kernel_fn_table(std::make_integer_sequence<int, kNumKernels>{})) kKernelFns{};

// Per-device address of g_tile_queues (hipGetSymbolAddress with the device
// current), and the launch sequence that picks the queue slot.
constexpr int kMaxDevices = 64;
std::atomic<unsigned long long *> g_queue_base[kMaxDevices];
std::atomic<unsigned long long> g_launch_seq{0};

unsigned long long *queue_base(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  unsigned long long *ptr = g_queue_base[device].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    void *addr = nullptr;
    if (hipGetSymbolAddress(&addr, HIP_SYMBOL(g_tile_queues)) != hipSuccess || addr == nullptr) return nullptr;
    ptr = (unsigned long long *)addr;
    g_queue_base[device].store(ptr, std::memory_order_release);
  }
  return ptr;
}

// CU count per device, asked once (the attribute query costs about a
// microsecond, a sizeable part of a launch).
std::atomic<int> g_cu_count[kMaxDevices];

int device_cu_count(int device) {
  if (device < 0 || device >= kMaxDevices) return kDefaultCuCount;
  int n = g_cu_count[device].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || n <= 0)
      n = kDefaultCuCount;
    g_cu_count[device].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace

// Split-KV partial results of fa_fwd_split_static: a library-owned buffer of
// FA_STATIC_SCRATCH_BYTES per device (held until the process ends), for
// callers that cannot allocate.  Every call on a device shares it; each call
// writes every partial it later reads (all KV runs of every row < Sq), so
// nothing needs clearing between calls.  In host code `scratch` names a
// host-side stand-in: the device address comes from hipGetSymbolAddress.
static __device__ __align__(256) char scratch[FA_STATIC_SCRATCH_BYTES];

namespace {

// Device address of `scratch`, asked once per device with that device
// current (each device holds its own copy of the array).
std::atomic<char *> g_scratch_base[kMaxDevices];

char *static_scratch_base(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  char *ptr = g_scratch_base[device].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    void *addr = nullptr;
    if (hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)) != hipSuccess || addr == nullptr) return nullptr;
    ptr = (char *)addr;
    g_scratch_base[device].store(ptr, std::memory_order_release);
  }
  return ptr;
}

}  // namespace

#ifdef FA_TIMING
static uint32_t *g_timing_buffer = nullptr;
extern "C" void fa_set_timing_buffer(void *p) { g_timing_buffer = (uint32_t *)p; }
#else
static uint32_t *const g_timing_buffer = nullptr;
#endif

namespace {

int launch(const fa_fwd_params *p, void *hip_stream, int splits, void *workspace, int64_t workspace_bytes) {
  const int rc = fa_validate(p);
  if (rc != FA_OK) return rc;
  if (p->B == 0 || p->H == 0 || p->Sq == 0) return FA_OK;
  int device = 0;
  const int cu_count = hipGetDevice(&device) == hipSuccess ? device_cu_count(device) : kDefaultCuCount;
  Plan plan;
  const int prc = make_plan(p, &plan, cu_count, splits);
  if (prc != FA_OK) return prc;
  const KernelMeta &e = kKernelMeta[plan.kernel];
  if (splits > 1) {
    if (!e.splittable) return FA_ERR_TILING;
    if (workspace == nullptr) return FA_ERR_NULL;
    if (((uintptr_t)workspace & 255u) != 0) return FA_ERR_ALIGN;
    const int64_t need = split_workspace_bytes(p, splits);
    if (need < 0 || workspace_bytes < need) return FA_ERR_SHAPE;
  }

  KernelArgs a;
  a.q = (const char *)p->q;
  a.k = (const char *)p->k;
  a.v = (const char *)p->v;
  a.o = (char *)p->o;
  a.lse = p->lse;
  a.q_sb = p->q_stride[0]; a.q_sh = p->q_stride[1]; a.q_ss = p->q_stride[2];
  a.k_sb = p->k_stride[0]; a.k_sh = p->k_stride[1]; a.k_ss = p->k_stride[2];
  a.v_sb = p->v_stride[0]; a.v_sh = p->v_stride[1]; a.v_ss = p->v_stride[2];
  a.o_sb = p->o_stride[0]; a.o_sh = p->o_stride[1]; a.o_ss = p->o_stride[2];
  a.B = p->B;
  a.H = p->H;
  a.Sq = p->Sq;
  a.Sk = p->Sk;
  a.n_mtiles = plan.n_mtiles;
  a.total_tiles = (int32_t)plan.total_tiles;
  a.kv_splits = splits > 1 ? splits : 1;
  a.split_tiles = splits > 1 ? plan.split_tiles : (1 << 30);
  a.part_o = splits > 1 ? (float *)workspace : nullptr;
  a.part_lse = splits > 1 ? (float *)((char *)workspace + split_part_o_bytes(p, splits)) : nullptr;
  hipStream_t stream = (hipStream_t)hip_stream;
  {
    // A launch recorded into a graph takes no counters (static schedule, see
    // TileQueue); an eager one takes the next launch slot.  A failed query
    // is treated as capture: the static schedule is always safe.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const bool capturing = hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone;
    if (capturing) {
      a.queue = nullptr;
    } else {
      unsigned long long *base = queue_base(device);
      if (base == nullptr) return FA_ERR_LAUNCH;
      const unsigned long long seq = g_launch_seq.fetch_add(1, std::memory_order_relaxed);
      a.queue = base + (seq % kQueueSlots) * kQueues * kQueueStride;
    }
    const int64_t bh = (int64_t)p->B * p->H;
    int64_t nq = kQueues;
    if (nq > plan.grid) nq = plan.grid;
    if (nq > bh) nq = bh;
    a.nq = (int32_t)nq;
    // Queue order: a queue's heads in groups of 8, each group's tiles
    // heaviest first across its heads, one band.  Measured on the benchmark
    // workloads against groups of 2..64 heads and 1..4 bands: within 1% of
    // the best time on each, with the least HBM traffic or close to it
    // (e.g. B8 H32 S3000 causal: 646 us and 2.5 GB fetched per launch, against
    // 804 us and 6.6 GB for all 32 heads of a queue at once; B16 H16 S1024:
    // 87 us against 101 us).
    const int64_t nh = (bh + nq - 1) / nq;  // heads of queue 0
    a.q_group = (int32_t)(nh < 8 ? (nh > 0 ? nh : 1) : 8);
    a.q_bands = 1;
  }
  // A negative scale is folded into Q (sign flip of every element, exact),
  // a zero scale into a tiny positive one (all logits ~0: uniform weights).
  const float s = p->sm_scale;
  a.q_sign = s < 0.f ? 0x80008000u : 0u;
  float c = fabsf(s) * kLog2e;
  if (c < 1e-30f) c = 1e-30f;
  a.c = c;
  a.timing = g_timing_buffer;

  hipLaunchKernelGGL(kKernelFns.fns[plan.kernel], dim3(plan.grid), dim3(64 * e.NW), (size_t)kernel_dyn_lds_bytes(e),
                     stream, a);
  if (hipGetLastError() != hipSuccess) return FA_ERR_LAUNCH;
  if (splits > 1) {
    MergeArgs m;
    m.part_o = a.part_o;
    m.part_lse = a.part_lse;
    m.o = a.o;
    m.lse = a.lse;
    m.o_sb = a.o_sb; m.o_sh = a.o_sh; m.o_ss = a.o_ss;
    m.B = p->B; m.H = p->H; m.Sq = p->Sq; m.D = p->D; m.splits = splits;
    const int64_t rows = (int64_t)p->B * p->H * p->Sq;
    const int64_t rows_per_block = 1024 / p->D;  // D / 4 lanes per row, 256 lanes
    const unsigned blocks = (unsigned)((rows + rows_per_block - 1) / rows_per_block);
    if (out_is_bf16(p->dtype)) {
      hipLaunchKernelGGL(fa_merge_kernel<true>, dim3(blocks), dim3(256), 0, stream, m);
    } else {
      hipLaunchKernelGGL(fa_merge_kernel<false>, dim3(blocks), dim3(256), 0, stream, m);
    }
    if (hipGetLastError() != hipSuccess) return FA_ERR_LAUNCH;
  }
  return FA_OK;
}

}  // namespace

extern "C" {

int fa_fwd(const fa_fwd_params *p, void *hip_stream) { return launch(p, hip_stream, 1, nullptr, 0); }

int fa_fwd_split(const fa_fwd_params *p, int32_t kv_splits, void *workspace, int64_t workspace_bytes,
                 void *hip_stream) {
  if (kv_splits < 1 || kv_splits > kMaxKvSplits) return FA_ERR_GRID;
  return launch(p, hip_stream, kv_splits, workspace, workspace_bytes);
}

int fa_fwd_split_static(const fa_fwd_params *p, int32_t kv_splits, void *hip_stream) {
  if (kv_splits < 1 || kv_splits > kMaxKvSplits) return FA_ERR_GRID;
  const int rc = fa_validate(p);
  if (rc != FA_OK) return rc;
  if (kv_splits == 1) return launch(p, hip_stream, 1, nullptr, 0);
  const int64_t need = split_workspace_bytes(p, kv_splits);
  if (need < 0 || need > (int64_t)FA_STATIC_SCRATCH_BYTES) return FA_ERR_SCRATCH;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return FA_ERR_LAUNCH;
  char *base = static_scratch_base(device);
  if (base == nullptr) return FA_ERR_LAUNCH;
  return launch(p, hip_stream, kv_splits, base, (int64_t)FA_STATIC_SCRATCH_BYTES);
}

}  // extern "C"
