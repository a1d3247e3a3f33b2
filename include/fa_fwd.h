/*
 * fa_fwd.h -- C ABI of the MI355X (gfx950) FlashAttention forward library
 * libfa_mi355x.so.
 *
 * This boundary replaces, one for one, the single host->device crossing of
 * the reference operator: the Triton launch `_attn_fwd[grid](...)` issued by
 * `_launch_kernel()` (flash_attention_forward.py:1130-1194, launch at
 * :1159-1193), together with the argument checks of `_validate_inputs()`
 * (:1114-1122), the tile resolution of `_resolve_tiling()` (:626-631) and the
 * runtime description of `_describe_runtime()` (:634-644).
 *
 * Conventions
 *  - Every tensor pointer is a DEVICE pointer owned by the caller.  The
 *    library allocates nothing and launches on the stream it is given.
 *  - Device state: the persistent grid pulls its tiles from queue counters
 *    in a library-owned __device__ array (per device: 1024 launch slots of
 *    8 counters).  An eager launch takes the next slot and leaves its
 *    counters at zero when it completes, so at most 1023 eager launches may
 *    be queued or running on one device at a time, over all streams and
 *    threads; more would share counters and race.  A launch made while its
 *    stream is capturing (graph) uses no counters (a static tile schedule),
 *    so graph replays share no device state with each other or with eager
 *    launches.
 *    fa_fwd_split_static also keeps its split-KV partial results in a
 *    library-owned __device__ buffer (see there).
 *  - Host state: a launch sequence number and per-device caches (CU count,
 *    counter and scratch addresses), all atomic: calls may come from any
 *    thread.
 *  - Strides are in ELEMENTS, in (batch, head, seq, dim) order.  The dim
 *    stride must be 1; the other strides must be non-negative multiples of 8
 *    elements, the seq stride at least D when the sequence has more than one
 *    row, and the base pointers 16-byte aligned (128-bit loads and stores).
 *    One (batch, head) slice of a tensor must span less than 2 GiB.
 *  - q, k and o share one element type, fp16 or bf16; v has that type too,
 *    or is fp8-e5m2 (FA_DTYPE_*_V_E5M2, every head dim; v strides then
 *    multiples of 16 elements).  lse is fp32,
 *    contiguous [B, H, Sq], natural log, over the scaled logits
 *    (lse[i] = log(sum_j exp(sm_scale * q_i . k_j)) over the visible keys),
 *    matching the reference's `m_i += log(l_i)` store at
 *    flash_attention_forward.py:1022,1031.  lse may be NULL.
 *  - Causal masking is top-left aligned: key j is visible to query i iff
 *    j <= i (flash_attention_forward.py:694-696; evaluate_attention.py:137-141).
 *  - Functions return 0 on success and a negative FA_ERR_* code on failure;
 *    no exception crosses the ABI.
 */
#ifndef FA_FWD_H
#define FA_FWD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA_ABI_VERSION 1

enum fa_dtype {
  FA_DTYPE_FP16 = 0,
  FA_DTYPE_BF16 = 1,
  /* v is fp8-e5m2 (OCP), q/k/o fp16 or bf16: P is rounded to e5m2 before
   * P.V, as the reference does when V.dtype is float8e5
   * (flash_attention_forward.py:704, :737, :996). */
  FA_DTYPE_FP16_V_E5M2 = 2,
  FA_DTYPE_BF16_V_E5M2 = 3,
};

enum fa_status {
  FA_OK = 0,
  FA_ERR_NULL = -1,        /* a required pointer is NULL                         */
  FA_ERR_SHAPE = -2,       /* negative size, Sq>0 with Sk==0, size overflow       */
  FA_ERR_HEAD_DIM = -3,    /* head dim not in the supported set                   */
  FA_ERR_DTYPE = -4,       /* dtype is not an enum fa_dtype value                 */
  FA_ERR_STRIDE = -5,      /* dim stride != 1 or a stride not a multiple of 8     */
  FA_ERR_ALIGN = -6,       /* a base pointer is not 16-byte aligned               */
  FA_ERR_TILING = -7,      /* block_m/block_n/num_waves: unsupported combination  */
  FA_ERR_SCALE = -8,       /* sm_scale is NaN or infinite                         */
  FA_ERR_GRID = -9,        /* persistent grid size is negative                    */
  FA_ERR_SCRATCH = -10,    /* split workspace larger than FA_STATIC_SCRATCH_BYTES */
  FA_ERR_LAUNCH = -100,    /* the HIP runtime rejected the launch                 */
};

/* One forward call.  Mirrors the arguments of the reference launch
 * (flash_attention_forward.py:1159-1193): Q, K, V, M (=lse), Out, sm_scale,
 * the 16 strides, Z, H, N_CTX, HEAD_DIM, BLOCK_M, BLOCK_N, STAGE (=causal). */
typedef struct fa_fwd_params {
  const void *q;
  const void *k;
  const void *v;
  void *o;
  float *lse;                 /* may be NULL: LSE is then not written */
  int64_t q_stride[4];
  int64_t k_stride[4];
  int64_t v_stride[4];
  int64_t o_stride[4];
  int32_t B, H, Sq, Sk, D;    /* the reference requires Sq == Sk; the kernel does not */
  int32_t dtype;              /* enum fa_dtype; o has the type of q and k */
  int32_t causal;             /* 0 or 1 */
  float sm_scale;
  int32_t block_m;            /* 0 = library default for (D, dtype, causal, S) */
  int32_t block_n;            /* 0 = library default; must be given with block_m */
  int32_t num_programs;       /* 0 = one workgroup per tile; >0 = persistent grid
                                 capped at this many workgroups (the reference's
                                 PERSISTENT_PROGRAMS, flash_attention_forward.py:616-623) */
} fa_fwd_params;

/* Slots of fa_query_config's output array. */
enum fa_config_slot {
  FA_CFG_BLOCK_M = 0,
  FA_CFG_BLOCK_N = 1,
  FA_CFG_WAVES = 2,
  FA_CFG_GRID = 3,           /* workgroups launched                          */
  FA_CFG_TOTAL_TILES = 4,    /* ceil(Sq / BLOCK_M) * B * H                    */
  FA_CFG_LDS_BYTES = 5,      /* LDS per workgroup                             */
  FA_CFG_STAGE = 6,          /* 3 causal, 1 non-causal (reference STAGE)      */
  FA_CFG_KERNEL_ID = 7,      /* index into the library's kernel table         */
  FA_CFG_COUNT = 8,
};

/* Launch the forward on `hip_stream` (a hipStream_t; NULL = default stream).
 * Asynchronous: returns once the launch is queued.  Replaces
 * `_attn_fwd[grid](...)` at flash_attention_forward.py:1159-1193. */
int fa_fwd(const fa_fwd_params *p, void *hip_stream);

/* Host-only argument check (no HIP call; usable without a GPU).  Replaces
 * `_validate_inputs` (flash_attention_forward.py:1114-1122) and the BM/BN
 * pairing check of `_resolve_tiling` (:627-628). */
int fa_validate(const fa_fwd_params *p);

/* Host-only: the kernel configuration fa_fwd would launch for *p, written to
 * out[FA_CFG_COUNT].  Replaces `_describe_runtime` (:634-644). */
int fa_query_config(const fa_fwd_params *p, int32_t out[FA_CFG_COUNT]);

/* Static string for a status code. */
const char *fa_error_string(int code);

/* FA_ABI_VERSION of the loaded library. */
int fa_abi_version(void);

/* Number of kernel instances in the library and a description of entry i:
 * out = {D, dtype, causal, BLOCK_M, BLOCK_N, waves}.  Host-only; lets the
 * tile sweep enumerate what it may pass as block_m/block_n. */
int fa_num_kernels(void);
int fa_kernel_info(int index, int32_t out[6]);

/* Resident workgroups per CU of kernel entry `index` (what its registers and
 * LDS allow; the persistent grid launches that many per CU), or FA_ERR_TILING
 * for an index out of range.  Host-only; the tile sweep records it with each
 * (BLOCK_M, BLOCK_N) candidate. */
int fa_kernel_wg_per_cu(int index);

/* Hash of the sources the library was compiled from (kernel source and this
 * header), as the build recipe computed it, or "unknown" for a build made
 * without it.  Host-only; lets a caller detect a library older than its
 * sources. */
const char *fa_build_id(void);

/* sizeof(fa_fwd_params) as compiled into the library, so a foreign binding
 * (ctypes, cffi) can check its struct layout before the first call. */
int fa_params_size(void);

/* ---- Split-KV.  No counterpart in the reference (its grid is one program per
 * (z, h, m-tile), flash_attention_forward.py:1125-1127).  For shapes whose
 * (head, m-tile) tiles leave most of the GPU idle (few heads, long sequences),
 * every m-tile's KV range is cut into kv_splits runs computed in parallel;
 * each run writes a partial O (fp32, normalised by its own row sum) and its
 * LSE into `workspace`, and a merge kernel combines them on the same stream:
 *     LSE = m + ln sum_s exp(LSE_s - m),  O = sum_s exp(LSE_s - LSE) O_s.
 * Results match fa_fwd within rounding (the sums are grouped differently). */

/* Workspace bytes fa_fwd_split needs for kv_splits (0 when kv_splits == 1);
 * negative FA_ERR_* on bad arguments. */
int64_t fa_split_workspace_bytes(const fa_fwd_params *p, int32_t kv_splits);

/* fa_fwd with the KV range split kv_splits ways (1 <= kv_splits <= 64).
 * workspace: device memory of at least fa_split_workspace_bytes bytes,
 * 256-byte aligned, owned by the caller and not read after the call's work
 * completes on the stream.  FA_ERR_TILING if the selected kernel cannot split. */
int fa_fwd_split(const fa_fwd_params *p, int32_t kv_splits, void *workspace, int64_t workspace_bytes,
                 void *hip_stream);

/* The library's split choice for these parameters: > 1 only when the
 * unsplit grid has at most one (head, m-tile) tile per two CUs; the runs then
 * fill one workgroup per CU (two for a causal mask), each keeping at least
 * 65536 key-columns (Sk / splits * D).  Host-only. */
int32_t fa_default_kv_splits(const fa_fwd_params *p);

/* ---- No-allocation split-KV.  No counterpart in the reference.  For callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc): fa_fwd_split with the
 * partial results in a library-owned static device buffer of
 * FA_STATIC_SCRATCH_BYTES per device (held until the process ends) instead of
 * a caller workspace; it calls no allocator.  FA_ERR_SCRATCH when
 * fa_split_workspace_bytes(p, kv_splits) exceeds the buffer.  Calls that
 * overlap on one device (any streams, including graph replays) share the
 * buffer and race: serialise them.  kv_splits == 1 is fa_fwd. */
#define FA_STATIC_SCRATCH_BYTES (32 * 1024 * 1024)
int fa_fwd_split_static(const fa_fwd_params *p, int32_t kv_splits, void *hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* FA_FWD_H */
