// fa_plan.cpp -- host-only half of libfa_mi355x.so: the kernel table's
// metadata, tile planning and the C-ABI calls that make no HIP call
// (fa_validate, fa_query_config, fa_default_kv_splits,
// fa_split_workspace_bytes, fa_kernel_info, fa_kernel_wg_per_cu, ...).
//
// Plain C++17 with no HIP header: fa_fwd.hip includes this file (the library
// stays one translation unit, and the kernel pointer table there is built
// from kKernelMeta below, entry for entry), and the host sanitizer test
// compiles it on its own with g++ -fsanitize=address,undefined.
//
// Counterparts in the reference (flash_attention_forward.py): argument checks
// of `_validate_inputs` (:1114-1122), the tile resolution of `_default_tiling`
// / `_resolve_tiling` (:221-242, :626-631), the grid of `_build_grid` and
// `_get_persistent_programs` (:616-623, :1125-1127), and `_describe_runtime`
// (:634-644).
#include <math.h>
#include <stdint.h>

#include "fa_fwd.h"

namespace {

// Rows a kernel may address past a tensor's end (a last partial m-tile, or the
// DMAs issued past the last KV tile); >= every BLOCK_M and ring depth * BLOCK_N.
constexpr int kRowMargin = 1024;

constexpr bool is_supported_head_dim(int d) { return d == 16 || d == 32 || d == 64 || d == 128 || d == 256; }
constexpr bool is_valid_dtype(int dt) {
  return dt == FA_DTYPE_FP16 || dt == FA_DTYPE_BF16 || dt == FA_DTYPE_FP16_V_E5M2 || dt == FA_DTYPE_BF16_V_E5M2;
}
constexpr bool v_is_fp8(int dt) { return dt == FA_DTYPE_FP16_V_E5M2 || dt == FA_DTYPE_BF16_V_E5M2; }
constexpr bool out_is_bf16(int dt) { return dt == FA_DTYPE_BF16 || dt == FA_DTYPE_BF16_V_E5M2; }
// Head dims of the fp8-V kernels.
constexpr bool is_supported_fp8v_head_dim(int d) { return is_supported_head_dim(d); }

// ---------------------------------------------------------------------------
// Kernel table metadata.  Two kernel families (fa_fwd.hip):
//  * kDma: fa_fwd_dma_kernel<D, BN, NW, stages, wg_per_cu, bf16, causal, fp8 V>,
//    4 waves (BLOCK_M 128), K/V through a 2-stage LDS ring filled by DMA;
//  * kPingPong: fa_fwd_pp_kernel<D, BN, stages, bf16, causal>, 8 waves
//    (BLOCK_M 256) in two phase-shifted groups, separate K and V rings of
//    `stages` tiles, one workgroup per CU, no split-KV.
enum KernelKind : int32_t { kDma = 0, kPingPong = 1 };

struct KernelMeta {
  int32_t kind;
  int32_t D, dtype, causal, BN, NW;
  int32_t stages;     // LDS stages of the K/V ring (ping-pong: per ring)
  int32_t wg_per_cu;  // resident workgroups per CU (registers and LDS)
  bool splittable;    // supports split-KV (partial outputs + merge)
};

// Dynamic LDS bytes of one workgroup: the Q area of the kernels with one
// workgroup per CU, 16-bit V and fewer 1 KB DMA chunks per wave than 32 Q rows
// fill (BLOCK_M rows of 2 D bytes); 0 for the others.
constexpr int32_t kernel_dyn_lds_bytes(const KernelMeta &m) {
  if (m.kind == kPingPong || m.wg_per_cu != 1 || v_is_fp8(m.dtype)) return 0;
  const int32_t ndma = 2 * (m.BN * 2 * m.D / 1024 / m.NW);  // K and V chunks per wave and tile
  return ndma < m.D / 16 ? 32 * m.NW * 2 * m.D : 0;
}

// LDS bytes of one workgroup (what the kernels' __shared__ arrays and the
// dynamic Q area add up to; fa_fwd.hip checks every entry against its
// kernel's own layout).
constexpr int32_t kernel_lds_bytes(const KernelMeta &m) {
  if (m.kind == kPingPong) return 2 * m.stages * m.BN * 2 * m.D;  // K and V rings
  const int32_t k_tile = m.BN * 2 * m.D;
  const int32_t v_tile = m.BN * (v_is_fp8(m.dtype) ? 1 : 2) * m.D;
  const int32_t v_ipt = v_tile / 1024;  // 1 KB DMA instructions per V tile
  const int32_t v_ipw = v_ipt >= m.NW ? v_ipt / m.NW : 1;
  return m.stages * (k_tile + v_ipw * m.NW * 1024) + kernel_dyn_lds_bytes(m);
}

constexpr KernelMeta dma(int D, int BN, int occ, int dtype, int causal) {
  return KernelMeta{kDma, D, dtype, causal, BN, 4, 2, occ, true};
}
constexpr KernelMeta pp(int D, int BN, int rings, int dtype, int causal) {
  return KernelMeta{kPingPong, D, dtype, causal, BN, 8, rings, 1, false};
}

#define FA_DMA4(D, BN, OCC)                                                                     \
  dma(D, BN, OCC, FA_DTYPE_FP16, 0), dma(D, BN, OCC, FA_DTYPE_FP16, 1), dma(D, BN, OCC, FA_DTYPE_BF16, 0), \
      dma(D, BN, OCC, FA_DTYPE_BF16, 1)
#define FA_PP4(D, BN, NR) \
  pp(D, BN, NR, FA_DTYPE_FP16, 0), pp(D, BN, NR, FA_DTYPE_FP16, 1), pp(D, BN, NR, FA_DTYPE_BF16, 0), pp(D, BN, NR, FA_DTYPE_BF16, 1)
// fp8-e5m2 V with fp16 / bf16 Q, K, O (dtype codes FA_DTYPE_*_V_E5M2).
#define FA_DMA8_4(D, BN, OCC)                                                                             \
  dma(D, BN, OCC, FA_DTYPE_FP16_V_E5M2, 0), dma(D, BN, OCC, FA_DTYPE_FP16_V_E5M2, 1),                   \
      dma(D, BN, OCC, FA_DTYPE_BF16_V_E5M2, 0), dma(D, BN, OCC, FA_DTYPE_BF16_V_E5M2, 1)

// The first entry matching (D, dtype, causal, BLOCK_N, waves) serves a launch.
constexpr KernelMeta kKernelMeta[] = {
    FA_DMA4(128, 64, 2),
    FA_PP4(128, 64, 4),
    // D = 128, 32-key tiles: the non-causal default, at three workgroups per
    // CU (1.5-3.7% faster than two, and equal to or up to 3.3% faster than
    // 64-key tiles at two); the causal kernel spills at three and keeps two.
    dma(128, 32, 3, FA_DTYPE_FP16, 0), dma(128, 32, 2, FA_DTYPE_FP16, 1),
    dma(128, 32, 3, FA_DTYPE_BF16, 0), dma(128, 32, 2, FA_DTYPE_BF16, 1),
    // D <= 64 is softmax (VALU) bound, and a single wave issues VALU work
    // well below the SIMD's rate: more resident waves fill the gaps.  D = 64
    // default: 64-key tiles, whose 32 KB of LDS and <= 168 registers let three
    // workgroups share a CU (0.7-7.7% faster than 128-key tiles at two, on
    // every D = 64 workload measured, fp16 and bf16, causal and not).
    FA_DMA4(64, 64, 3),
    FA_PP4(64, 64, 4),
    FA_DMA4(64, 32, 2),
    FA_DMA4(64, 128, 2),
    // D = 256: 512 registers per wave (O^T alone is 128), so one workgroup
    // per CU; 32-key tiles keep S, P and the operand fragments small.  The
    // 64-key kernels are candidates for the tile sweep.
    FA_DMA4(256, 32, 1),
    FA_DMA4(256, 64, 1),
    // D = 32: four workgroups per CU when causal (8-9% faster than two);
    // non-causal measured 1.7% slower at four, so it keeps two.
    dma(32, 64, 2, FA_DTYPE_FP16, 0), dma(32, 64, 4, FA_DTYPE_FP16, 1),
    dma(32, 64, 2, FA_DTYPE_BF16, 0), dma(32, 64, 4, FA_DTYPE_BF16, 1),
    // D = 16: a 64-key tile is only two DMA instructions; 128 keys give each
    // wave one.  Three workgroups per CU (4-10% faster than two).
    FA_DMA4(16, 128, 3),
    FA_DMA8_4(128, 64, 2),
    // fp8 V at D <= 64: three workgroups per CU (causal 6.7-8.4% faster than
    // two, non-causal equal).
    FA_DMA8_4(64, 64, 3),
    FA_DMA8_4(256, 64, 1),
    FA_DMA8_4(32, 64, 3),
    FA_DMA8_4(16, 128, 3),
};
#undef FA_DMA4
#undef FA_PP4
#undef FA_DMA8_4
constexpr int kNumKernels = sizeof(kKernelMeta) / sizeof(kKernelMeta[0]);

constexpr bool table_fits_lds() {
  for (const KernelMeta &m : kKernelMeta)
    if (kernel_lds_bytes(m) * m.wg_per_cu > 160 * 1024) return false;
  return true;
}
static_assert(table_fits_lds(), "LDS budget of one gfx950 CU");

// Default (BLOCK_N, waves) per head dim; BLOCK_M = 32 * waves.
void default_tiling(int D, int dtype, int causal, int *bn, int *nw) {
  // fp8 V: 64-key tiles (D = 16: 128), one 32x32x64 MFMA per 64 keys and 32
  // head dims.  16-bit V: 64 keys, except D = 16 (128), D = 256 (32) and
  // non-causal D = 128 (32, the three-workgroups-per-CU kernel).
  if (v_is_fp8(dtype))
    *bn = D == 16 ? 128 : 64;
  else if (D == 16)
    *bn = 128;
  else if (D == 256 || (D == 128 && !causal))
    *bn = 32;
  else
    *bn = 64;
  *nw = 4;
}

int find_kernel(int D, int dtype, int causal, int BN, int NW) {
  for (int i = 0; i < kNumKernels; ++i) {
    const KernelMeta &e = kKernelMeta[i];
    if (e.D == D && e.dtype == dtype && e.causal == causal && e.BN == BN && e.NW == NW) return i;
  }
  return -1;
}

struct Plan {
  int kernel;
  int BM, BN, NW;
  int n_mtiles;
  int64_t total_tiles;  // (head, m-tile) tiles
  int grid;
  int split_tiles;      // KV tiles per split-KV run (0: no split)
};

constexpr int kMaxKvSplits = 64;

// CUs of an MI355X; fa_fwd asks the device, the host-only calls assume this.
constexpr int kDefaultCuCount = 256;

int make_plan(const fa_fwd_params *p, Plan *out, int cu_count = kDefaultCuCount, int splits = 1) {
  int bn, nw;
  if (p->block_m == 0 && p->block_n == 0) {
    default_tiling(p->D, p->dtype, p->causal, &bn, &nw);
  } else {
    if (p->block_m <= 0 || p->block_n <= 0 || p->block_m % 32 != 0) return FA_ERR_TILING;
    bn = p->block_n;
    nw = p->block_m / 32;
  }
  const int kid = find_kernel(p->D, p->dtype, p->causal ? 1 : 0, bn, nw);
  if (kid < 0) return FA_ERR_TILING;
  out->kernel = kid;
  out->BN = bn;
  out->NW = nw;
  out->BM = 32 * nw;
  out->n_mtiles = (int)(((int64_t)p->Sq + out->BM - 1) / out->BM);
  const int64_t heads = (int64_t)p->B * p->H;  // < 2^62: no overflow
  if (heads > INT32_MAX) return FA_ERR_SHAPE;
  out->total_tiles = (int64_t)out->n_mtiles * heads;
  if (out->total_tiles > INT32_MAX) return FA_ERR_SHAPE;
  // Persistent grid: as many workgroups as fit on the GPU at once, pulling
  // tiles from the tile queues; PERSISTENT_PROGRAMS (num_programs) overrides
  // the count.
  const int64_t kv_tiles = ((int64_t)p->Sk + bn - 1) / bn;
  out->split_tiles = splits > 1 ? (int)((kv_tiles + splits - 1) / splits) : 0;
  const int64_t units = out->total_tiles * (splits > 1 ? splits : 1);
  if (units > INT32_MAX) return FA_ERR_SHAPE;
  int64_t grid = (int64_t)kKernelMeta[kid].wg_per_cu * (cu_count > 0 ? cu_count : kDefaultCuCount);
  if (p->num_programs > 0) grid = p->num_programs;
  if (grid > units) grid = units;
  out->grid = (int)grid;
  return FA_OK;
}

bool aligned16(const void *ptr) { return ((uintptr_t)ptr & 15u) == 0; }

// Workspace of a split-KV launch: partial O, then (256-byte aligned) LSE.
// Sizes are formed in 128-bit arithmetic; a workspace of 2^62 bytes or more
// (no device has one) is reported as -1.
constexpr __int128 kMaxWorkspace = (__int128)1 << 62;
int64_t split_part_o_bytes(const fa_fwd_params *p, int splits) {
  const __int128 b = ((__int128)splits * p->B * p->H * p->Sq * p->D * 4 + 255) / 256 * 256;
  return b < kMaxWorkspace ? (int64_t)b : -1;
}
int64_t split_workspace_bytes(const fa_fwd_params *p, int splits) {
  const int64_t po = split_part_o_bytes(p, splits);
  const __int128 b = (__int128)po + (__int128)splits * p->B * p->H * p->Sq * 4;
  return po >= 0 && b < kMaxWorkspace ? (int64_t)b : -1;
}

}  // namespace

#ifndef FA_SOURCE_HASH
#define FA_SOURCE_HASH "unknown"
#endif

extern "C" {

int fa_abi_version(void) { return FA_ABI_VERSION; }

const char *fa_build_id(void) { return FA_SOURCE_HASH; }

const char *fa_error_string(int code) {
  switch (code) {
    case FA_OK: return "ok";
    case FA_ERR_NULL: return "a required tensor pointer is NULL";
    case FA_ERR_SHAPE: return "invalid shape (negative size, Sq>0 with Sk==0, or too many tiles)";
    case FA_ERR_HEAD_DIM: return "HEAD_DIM is not one of 16, 32, 64, 128, 256";
    case FA_ERR_DTYPE: return "dtype must be fp16 or bf16 (optionally with fp8-e5m2 V)";
    case FA_ERR_STRIDE: return "the head-dim stride must be 1 and the other strides multiples of 8 elements (16 for an fp8 V)";
    case FA_ERR_ALIGN: return "tensor base pointers must be 16-byte aligned";
    case FA_ERR_TILING: return "unsupported BLOCK_M/BLOCK_N combination";
    case FA_ERR_SCALE: return "sm_scale must be finite";
    case FA_ERR_GRID: return "the persistent program count must be >= 0";
    case FA_ERR_SCRATCH: return "the split-KV partial results exceed the library's static scratch buffer (FA_STATIC_SCRATCH_BYTES)";
    case FA_ERR_LAUNCH: return "the HIP runtime rejected the kernel launch";
    default: return "unknown fa_fwd status";
  }
}

int fa_validate(const fa_fwd_params *p) {
  if (p == nullptr) return FA_ERR_NULL;
  if (p->B < 0 || p->H < 0 || p->Sq < 0 || p->Sk < 0 || p->D <= 0) return FA_ERR_SHAPE;
  if (p->Sq > 0 && p->Sk == 0 && p->B > 0 && p->H > 0) return FA_ERR_SHAPE;
  if (!is_supported_head_dim(p->D)) return FA_ERR_HEAD_DIM;
  if (!is_valid_dtype(p->dtype)) return FA_ERR_DTYPE;
  if (v_is_fp8(p->dtype) && !is_supported_fp8v_head_dim(p->D)) return FA_ERR_HEAD_DIM;
  if (!(p->sm_scale == p->sm_scale) || isinf(p->sm_scale)) return FA_ERR_SCALE;
  if (p->num_programs < 0) return FA_ERR_GRID;
  if ((p->block_m == 0) != (p->block_n == 0)) return FA_ERR_TILING;
  const bool empty = p->B == 0 || p->H == 0 || p->Sq == 0;
  if (empty) return FA_OK;
  if (p->q == nullptr || p->k == nullptr || p->v == nullptr || p->o == nullptr) return FA_ERR_NULL;
  const int64_t *st[4] = {p->q_stride, p->k_stride, p->v_stride, p->o_stride};
  const int64_t rows[4] = {p->Sq, p->Sk, p->Sk, p->Sq};
  for (int t = 0; t < 4; ++t) {
    // 16-byte rows: strides in multiples of 8 16-bit or 16 fp8 elements.
    const int64_t align = (t == 2 && v_is_fp8(p->dtype)) ? 16 : 8;
    if (st[t][3] != 1) return FA_ERR_STRIDE;
    for (int i = 0; i < 3; ++i)
      if (st[t][i] < 0 || st[t][i] % align != 0) return FA_ERR_STRIDE;
    if (rows[t] > 1 && st[t][2] < p->D) return FA_ERR_STRIDE;
    // Buffer offsets inside one (b, h) slice are 32-bit: keep the slice, plus
    // the rows past its end that a last partial m-tile or the DMAs issued past
    // the last KV tile address, below 2 GiB.  rows < 2^31 and row_stride <
    // 2^31 here, so the product is formed in 128-bit arithmetic (it can
    // exceed int64: e.g. 2^31 rows of a 2^31 - 8 element stride).
    const int64_t row_stride = st[t][2] > p->D ? st[t][2] : p->D;
    if (row_stride >= ((int64_t)1 << 31)) return FA_ERR_SHAPE;
    if ((__int128)(rows[t] + kRowMargin) * row_stride * 2 >= ((__int128)1 << 31)) return FA_ERR_SHAPE;
  }
  if ((int64_t)p->Sq * 4 >= ((int64_t)1 << 31)) return FA_ERR_SHAPE;
  if (!aligned16(p->q) || !aligned16(p->k) || !aligned16(p->v) || !aligned16(p->o)) return FA_ERR_ALIGN;
  if (p->lse != nullptr && ((uintptr_t)p->lse & 3u) != 0) return FA_ERR_ALIGN;
  Plan plan;
  return make_plan(p, &plan);
}

int fa_query_config(const fa_fwd_params *p, int32_t out[FA_CFG_COUNT]) {
  if (p == nullptr || out == nullptr) return FA_ERR_NULL;
  if (p->B < 0 || p->H < 0 || p->Sq < 0 || p->Sk < 0) return FA_ERR_SHAPE;
  if (!is_supported_head_dim(p->D)) return FA_ERR_HEAD_DIM;
  if (!is_valid_dtype(p->dtype)) return FA_ERR_DTYPE;
  if (v_is_fp8(p->dtype) && !is_supported_fp8v_head_dim(p->D)) return FA_ERR_HEAD_DIM;
  if ((p->block_m == 0) != (p->block_n == 0)) return FA_ERR_TILING;
  if (p->num_programs < 0) return FA_ERR_GRID;
  Plan plan;
  const int rc = make_plan(p, &plan);
  if (rc != FA_OK) return rc;
  out[FA_CFG_BLOCK_M] = plan.BM;
  out[FA_CFG_BLOCK_N] = plan.BN;
  out[FA_CFG_WAVES] = plan.NW;
  out[FA_CFG_GRID] = plan.grid;
  out[FA_CFG_TOTAL_TILES] = (int32_t)plan.total_tiles;
  out[FA_CFG_LDS_BYTES] = kernel_lds_bytes(kKernelMeta[plan.kernel]);
  out[FA_CFG_STAGE] = p->causal ? 3 : 1;
  out[FA_CFG_KERNEL_ID] = plan.kernel;
  return FA_OK;
}

int fa_num_kernels(void) { return kNumKernels; }

int fa_params_size(void) { return (int)sizeof(fa_fwd_params); }

int fa_kernel_info(int index, int32_t out[6]) {
  if (out == nullptr) return FA_ERR_NULL;
  if (index < 0 || index >= kNumKernels) return FA_ERR_TILING;
  const KernelMeta &e = kKernelMeta[index];
  out[0] = e.D;
  out[1] = e.dtype;
  out[2] = e.causal;
  out[3] = 32 * e.NW;
  out[4] = e.BN;
  out[5] = e.NW;
  return FA_OK;
}

int fa_kernel_wg_per_cu(int index) {
  if (index < 0 || index >= kNumKernels) return FA_ERR_TILING;
  return kKernelMeta[index].wg_per_cu;
}

int64_t fa_split_workspace_bytes(const fa_fwd_params *p, int32_t kv_splits) {
  if (p == nullptr) return FA_ERR_NULL;
  if (kv_splits < 1 || kv_splits > kMaxKvSplits) return FA_ERR_GRID;
  if (p->B < 0 || p->H < 0 || p->Sq < 0 || p->D <= 0) return FA_ERR_SHAPE;
  if (kv_splits == 1) return 0;
  const int64_t bytes = split_workspace_bytes(p, kv_splits);
  return bytes >= 0 ? bytes : (int64_t)FA_ERR_SHAPE;
}

int32_t fa_default_kv_splits(const fa_fwd_params *p) {
  // Shape-only (no pointer or stride checks): usable before tensors exist.
  if (p == nullptr || p->B <= 0 || p->H <= 0 || p->Sq <= 0 || p->Sk <= 0) return 1;
  if (!is_supported_head_dim(p->D) || !is_valid_dtype(p->dtype)) return 1;
  Plan plan;
  if (make_plan(p, &plan) != FA_OK) return 1;
  const KernelMeta &e = kKernelMeta[plan.kernel];
  if (!e.splittable) return 1;
  // Fitted to 25 shapes timed on MI355X with 1..8 splits (B1-2, H1-16,
  // S256-16384, D16-256, fp16):
  //  * only grids of at most half a workgroup per CU split: at one tile per
  //    CU (256) a second workgroup per CU gained nothing (B1 H8 S4096 D64:
  //    50 -> 54 us with 2 splits) or at most 3-5%;
  //  * the runs fill one workgroup per CU, two for causal grids, whose
  //    longest m-tile (all keys) sets the time while the others finish
  //    early (B1 H4 S4096 D128 causal: 62 -> 42 us at 2, 41 at 4);
  //  * each run keeps at least 64K key-columns (Sk / splits * D >= 65536):
  //    below that the merge launch and its HBM pass cost more than the
  //    shorter runs save (B1 H4 S1024 D64: 14.7 -> 15.7 us at 2 splits).
  // These picks were within 8% of the fastest split count on every shape
  // timed (18 of 25 the fastest), against up to 18% slower under the earlier
  // rule (at least 8 KV tiles and 512 keys a run, up to two workgroups per CU).
  if (plan.total_tiles * 2 > kDefaultCuCount) return 1;
  const int64_t fill = (p->causal ? 2 : 1) * kDefaultCuCount / plan.total_tiles;
  const int64_t work = (int64_t)p->Sk * p->D / 65536;
  int64_t splits = fill < work ? fill : work;
  if (splits > kMaxKvSplits) splits = kMaxKvSplits;
  return splits > 1 ? (int32_t)splits : 1;
}

}  // extern "C"
