// Host-only driver of the C ABI's planning calls, built together with
// flash_attn_npu_amd/csrc/fa_plan.cpp under AddressSanitizer and
// UndefinedBehaviorSanitizer by tests/test_host_sanitizers.py (no HIP, no GPU).
//
// It walks fa_validate, fa_query_config, fa_default_kv_splits,
// fa_split_workspace_bytes, fa_kernel_info, fa_kernel_wg_per_cu and
// fa_error_string over hand-picked edge cases and a seeded random sweep
// (sizes and strides up to their type limits, negative values, NULL
// pointers, odd alignments), and checks the invariants the Python layer
// relies on.  Any sanitizer report aborts the run (-fno-sanitize-recover);
// a broken invariant prints FAIL and exits 1.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "fa_fwd.h"

static int g_failures = 0;
#define CHECK(cond, ...)                                   \
  do {                                                     \
    if (!(cond)) {                                         \
      ++g_failures;                                        \
      fprintf(stderr, "FAIL %s:%d: %s: ", __FILE__, __LINE__, #cond); \
      fprintf(stderr, __VA_ARGS__);                        \
      fprintf(stderr, "\n");                               \
    }                                                      \
  } while (0)

static uint64_t g_rng = 0x9E3779B97F4A7C15ull;
static uint64_t next_u64() {  // splitmix64
  uint64_t z = (g_rng += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static const int32_t kI32Edges[] = {0, 1, 2, 7, 31, 32, 33, 63, 64, 127, 128, 129, 511, 512, 2048, 3000, 8192,
                                    65535, 1 << 20, INT32_MAX / 2, INT32_MAX - 1, INT32_MAX, -1, INT32_MIN};
static const int64_t kI64Edges[] = {0, 1, 8, 16, 64, 128, 256, 4096, 1 << 20, (int64_t)1 << 31,
                                    (int64_t)1 << 40, INT64_MAX / 2, INT64_MAX, -8, INT64_MIN};

static int32_t pick_i32() {
  const uint64_t r = next_u64();
  if (r % 3 == 0) return kI32Edges[(r >> 8) % (sizeof(kI32Edges) / sizeof(kI32Edges[0]))];
  return (int32_t)((r >> 16) % 5000);
}
static int64_t pick_i64(int64_t dense) {
  const uint64_t r = next_u64();
  if (r % 4 == 0) return kI64Edges[(r >> 8) % (sizeof(kI64Edges) / sizeof(kI64Edges[0]))];
  return dense * (int64_t)((r >> 16) % 3);
}

static void dense_strides(fa_fwd_params *p) {
  int64_t *st[4] = {p->q_stride, p->k_stride, p->v_stride, p->o_stride};
  const int64_t rows[4] = {p->Sq, p->Sk, p->Sk, p->Sq};
  for (int t = 0; t < 4; ++t) {
    st[t][3] = 1;
    st[t][2] = p->D;
    st[t][1] = rows[t] * p->D;
    st[t][0] = (int64_t)p->H * rows[t] * p->D;
  }
}

static fa_fwd_params valid_params(int B, int H, int S, int D, int dtype, int causal) {
  fa_fwd_params p;
  memset(&p, 0, sizeof p);
  // Fake, 16-byte-aligned device addresses: the host-only calls never dereference them.
  p.q = (const void *)(uintptr_t)0x100000000ull;
  p.k = (const void *)(uintptr_t)0x200000000ull;
  p.v = (const void *)(uintptr_t)0x300000000ull;
  p.o = (void *)(uintptr_t)0x400000000ull;
  p.lse = (float *)(uintptr_t)0x500000000ull;
  p.B = B;
  p.H = H;
  p.Sq = S;
  p.Sk = S;
  p.D = D;
  p.dtype = dtype;
  p.causal = causal;
  p.sm_scale = 0.125f;
  dense_strides(&p);
  return p;
}

static bool known_status(int rc) {
  return rc == FA_OK || (rc <= FA_ERR_NULL && rc >= FA_ERR_SCRATCH) || rc == FA_ERR_LAUNCH;
}

struct KernelRow {
  int32_t D, dtype, causal, BM, BN, NW, wg;
};

static void check_params(const fa_fwd_params &p, const KernelRow *rows, int nk) {
  const int v = fa_validate(&p);
  CHECK(known_status(v), "fa_validate returned %d", v);
  int32_t cfg[FA_CFG_COUNT];
  memset(cfg, 0x7f, sizeof cfg);
  const int q = fa_query_config(&p, cfg);
  CHECK(known_status(q), "fa_query_config returned %d", q);
  if (v == FA_OK && p.B > 0 && p.H > 0 && p.Sq > 0) {
    // Every call the library would launch has a configuration to describe.
    CHECK(q == FA_OK, "valid params but fa_query_config = %d", q);
  }
  if (q == FA_OK) {
    CHECK(cfg[FA_CFG_KERNEL_ID] >= 0 && cfg[FA_CFG_KERNEL_ID] < nk, "kernel id %d", cfg[FA_CFG_KERNEL_ID]);
    if (cfg[FA_CFG_KERNEL_ID] >= 0 && cfg[FA_CFG_KERNEL_ID] < nk) {
      const KernelRow &r = rows[cfg[FA_CFG_KERNEL_ID]];
      CHECK(r.D == p.D && r.dtype == p.dtype && r.causal == (p.causal ? 1 : 0), "kernel row mismatch");
      CHECK(cfg[FA_CFG_BLOCK_M] == r.BM && cfg[FA_CFG_BLOCK_N] == r.BN && cfg[FA_CFG_WAVES] == r.NW,
            "tiling %d/%d/%d vs row %d/%d/%d", cfg[0], cfg[1], cfg[2], r.BM, r.BN, r.NW);
      CHECK(cfg[FA_CFG_LDS_BYTES] > 0 && cfg[FA_CFG_LDS_BYTES] * r.wg <= 160 * 1024, "LDS %d x %d",
            cfg[FA_CFG_LDS_BYTES], r.wg);
    }
    CHECK(cfg[FA_CFG_BLOCK_M] == 32 * cfg[FA_CFG_WAVES], "BM != 32 * waves");
    CHECK((cfg[FA_CFG_GRID] >= 0 && cfg[FA_CFG_GRID] <= cfg[FA_CFG_TOTAL_TILES]) || cfg[FA_CFG_TOTAL_TILES] == 0,
          "grid %d > tiles %d", cfg[FA_CFG_GRID], cfg[FA_CFG_TOTAL_TILES]);
    CHECK(cfg[FA_CFG_STAGE] == (p.causal ? 3 : 1), "stage");
  }
  const int32_t splits = fa_default_kv_splits(&p);
  CHECK(splits >= 1 && splits <= 64, "default splits %d", splits);
  int64_t prev = 0;
  for (int32_t s = 0; s <= 66; s += (s < 4 ? 1 : 31)) {
    const int64_t b = fa_split_workspace_bytes(&p, s);
    if (s < 1 || s > 64) {
      CHECK(b == FA_ERR_GRID, "splits %d accepted (%lld)", s, (long long)b);
    } else if (s == 1) {
      CHECK(b == 0 || b < 0, "one split needs no workspace (%lld)", (long long)b);
    } else if (b >= 0) {
      CHECK(b >= prev, "workspace shrinks with more splits");
      CHECK(b % 4 == 0, "workspace %lld", (long long)b);
      prev = b;
    } else {
      CHECK(b == FA_ERR_SHAPE || b == FA_ERR_NULL, "workspace error %lld", (long long)b);
    }
  }
}

int main() {
  const int nk = fa_num_kernels();
  CHECK(nk > 0 && nk <= 1024, "%d kernels", nk);
  KernelRow rows[1024];
  for (int i = 0; i < nk && i < 1024; ++i) {
    int32_t out[6];
    CHECK(fa_kernel_info(i, out) == FA_OK, "kernel_info %d", i);
    rows[i] = KernelRow{out[0], out[1], out[2], out[3], out[4], out[5], fa_kernel_wg_per_cu(i)};
    CHECK(rows[i].wg >= 1 && rows[i].wg <= 4, "wg_per_cu %d", rows[i].wg);
    CHECK(rows[i].BM == 32 * rows[i].NW, "BM");
  }
  int32_t out6[6];
  CHECK(fa_kernel_info(-1, out6) == FA_ERR_TILING && fa_kernel_info(nk, out6) == FA_ERR_TILING, "index range");
  CHECK(fa_kernel_info(0, nullptr) == FA_ERR_NULL, "null out");
  CHECK(fa_kernel_wg_per_cu(-1) == FA_ERR_TILING && fa_kernel_wg_per_cu(nk) == FA_ERR_TILING, "wg range");
  CHECK(fa_params_size() == (int)sizeof(fa_fwd_params), "params size");
  CHECK(fa_abi_version() == FA_ABI_VERSION, "abi version");
  CHECK(fa_build_id() != nullptr && strlen(fa_build_id()) > 0, "build id");
  for (int code = -200; code <= 10; ++code) {
    const char *s = fa_error_string(code);
    CHECK(s != nullptr && strlen(s) > 0, "error string %d", code);
  }
  CHECK(fa_validate(nullptr) == FA_ERR_NULL, "validate(NULL)");
  int32_t cfg[FA_CFG_COUNT];
  CHECK(fa_query_config(nullptr, cfg) == FA_ERR_NULL, "query(NULL)");
  CHECK(fa_default_kv_splits(nullptr) == 1, "splits(NULL)");
  CHECK(fa_split_workspace_bytes(nullptr, 2) == FA_ERR_NULL, "workspace(NULL)");

  // Every kernel of the table, at the benchmark sizes and at ragged ones.
  const int dims[] = {16, 32, 64, 128, 256};
  const int seqs[] = {1, 37, 128, 512, 2048, 3000, 8192, 131072};
  for (int dt = 0; dt < 4; ++dt)
    for (int d : dims)
      for (int c = 0; c < 2; ++c)
        for (int s : seqs) {
          fa_fwd_params p = valid_params(2, 3, s, d, dt, c);
          CHECK(fa_validate(&p) == FA_OK, "D %d dtype %d causal %d S %d: %d", d, dt, c, s, fa_validate(&p));
          check_params(p, rows, nk);
          for (int i = 0; i < nk; ++i) {  // every BM/BN override of the matching kernels
            if (rows[i].D != d || rows[i].dtype != dt || rows[i].causal != c) continue;
            p.block_m = rows[i].BM;
            p.block_n = rows[i].BN;
            check_params(p, rows, nk);
            p.num_programs = 7;
            check_params(p, rows, nk);
            p.num_programs = 0;
          }
          p.block_m = 96;  // no such kernel
          p.block_n = 48;
          CHECK(fa_validate(&p) == FA_ERR_TILING, "odd tiling accepted");
        }

  // Slices near the 2 GiB limit: sequence lengths up to INT32_MAX with seq
  // strides just below 2^31 elements (the slice-size product exceeds int64).
  {
    const int64_t big_strides[] = {(int64_t)(1u << 31) - 8, (int64_t)1 << 30, 1 << 20, 128};
    const int big_seqs[] = {INT32_MAX, INT32_MAX - 1, 1 << 30, 1 << 24, 1000};
    for (int64_t ss : big_strides)
      for (int sk : big_seqs)
        for (int which = 0; which < 2; ++which) {
          fa_fwd_params p = valid_params(1, 1, 64, 128, 1, 1);
          if (which == 0) {
            p.Sk = sk;
            p.k_stride[2] = ss;
            p.v_stride[2] = ss;
          } else {
            p.Sq = sk;
            p.q_stride[2] = ss;
            p.o_stride[2] = ss;
          }
          const int v = fa_validate(&p);
          const bool fits = ((__int128)((int64_t)sk + 1024) * (ss > 128 ? ss : 128) * 2) < ((__int128)1 << 31);
          CHECK(v == (fits ? FA_OK : FA_ERR_SHAPE), "S %d stride %lld: %d", sk, (long long)ss, v);
          check_params(p, rows, nk);
        }
  }

  // Seeded random sweep over every field, including limits and garbage.
  for (int it = 0; it < 200000; ++it) {
    fa_fwd_params p = valid_params(1 + (int)(next_u64() % 8), 1 + (int)(next_u64() % 40),
                                   1 + (int)(next_u64() % 4096), dims[next_u64() % 5], (int)(next_u64() % 4),
                                   (int)(next_u64() % 2));
    const uint64_t what = next_u64();
    if (what & 1) p.B = pick_i32();
    if (what & 2) p.H = pick_i32();
    if (what & 4) p.Sq = pick_i32();
    if (what & 8) p.Sk = pick_i32();
    if (what & 16) p.D = pick_i32() % 300;
    if (what & 32) p.dtype = (int32_t)(next_u64() % 7) - 1;
    if (what & 64) p.causal = (int32_t)(next_u64() % 3);
    if (what & 128) {
      int64_t *st[4] = {p.q_stride, p.k_stride, p.v_stride, p.o_stride};
      int64_t *s = st[next_u64() % 4];
      s[next_u64() % 4] = pick_i64(s[2]);
    }
    if (what & 256) {
      p.block_m = (int32_t)(next_u64() % 5) * 64;
      p.block_n = (int32_t)(next_u64() % 5) * 32;
    }
    if (what & 512) p.num_programs = pick_i32();
    if (what & 1024) p.q = (const void *)(uintptr_t)(0x100000000ull + next_u64() % 32);
    if (what & 2048) p.lse = (what & 4096) ? nullptr : (float *)(uintptr_t)(0x500000002ull);
    if (what & 8192) {
      const float bad[] = {0.f, -0.5f, 1e30f, __builtin_inff(), __builtin_nanf("")};
      p.sm_scale = bad[next_u64() % 5];
    }
    if (what & 16384) p.o = nullptr;
    check_params(p, rows, nk);
  }
  if (g_failures) {
    fprintf(stderr, "%d invariant failures\n", g_failures);
    return 1;
  }
  printf("abi host check ok: %d kernels\n", nk);
  return 0;
}
