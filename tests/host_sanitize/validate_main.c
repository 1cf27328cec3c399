/*
 * Host-side validation of the C ABI under AddressSanitizer and
 * UndefinedBehaviorSanitizer (tests/test_host_sanitize.py builds and runs it;
 * no GPU is needed).  Every entry point of include/ssa_mi355x.h and
 * include/ssa_decoder_ops.h is called with NULL arguments, with each integer
 * field set to 0, -1, INT32_MIN and INT32_MAX in turn, and with each stride set
 * to negative, unaligned and huge values; the size queries get the same
 * extremes.  Pointers are never dereferenced on the host, and every call that
 * passes validation reaches a kernel launch, which fails without a device; so
 * what is checked is that validation and the host arithmetic behind it have no
 * undefined behaviour (signed overflow, bad shifts, out-of-bounds reads) for
 * any argument values, plus the status codes of known-bad arguments.  The
 * pointers are fake, so the program refuses to run where a GPU is visible.
 */
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../../include/ssa_decoder_ops.h"
#include "../../include/ssa_mi355x.h"

#define FAKE ((void*)(uintptr_t)0x100000)

/* HIP runtime (libamdhip64): hipError_t is an int-sized enum, hipSuccess = 0 */
int hipGetDeviceCount(int* count);

static int failures = 0;
static long calls = 0;

static void expect(int got, int want, const char* what) {
  if (got != want) {
    fprintf(stderr, "FAIL %s: status %d, expected %d\n", what, got, want);
    ++failures;
  }
}

static const int32_t kInts[] = {0, -1, INT32_MIN, INT32_MAX, 1 << 30};
static const int64_t kStrides[] = {-8, INT64_MIN, INT64_MAX & ~(int64_t)7, (int64_t)1 << 24, 4, (int64_t)1 << 40};
#define NI ((int)(sizeof(kInts) / sizeof(kInts[0])))
#define NS ((int)(sizeof(kStrides) / sizeof(kStrides[0])))

static ssa_tensor4 t4(int64_t sh, int64_t ss) {
  ssa_tensor4 t = {FAKE, 8 * sh, sh, ss};
  return t;
}

static ssa_fwd_args base_fwd(void) {
  ssa_fwd_args a;
  memset(&a, 0, sizeof a);
  a.q = a.out = t4(256 * 128, 128);
  a.k = a.v = t4(256 * 128, 128);
  a.m = (float*)FAKE;
  a.ssa_n = a.ssa_b = (const float*)FAKE;
  a.batch = 2, a.heads_q = 8, a.heads_kv = 2, a.seqlen = 256, a.head_dim = 128;
  a.dtype = SSA_DTYPE_BF16, a.causal = 1, a.softmax_scale = 0.088f;
  return a;
}

static ssa_bwd_args base_bwd(void) {
  ssa_bwd_args a;
  memset(&a, 0, sizeof a);
  a.q = a.out = a.dout = a.dq = t4(256 * 128, 128);
  a.k = a.v = a.dk = a.dv = t4(256 * 128, 128);
  a.m = (const float*)FAKE;
  a.delta = a.partials = a.dn = a.db = (float*)FAKE;
  a.ssa_n = a.ssa_b = (const float*)FAKE;
  a.batch = 2, a.heads_q = 8, a.heads_kv = 2, a.seqlen = 256, a.head_dim = 128;
  a.dtype = SSA_DTYPE_BF16, a.causal = 1, a.softmax_scale = 0.088f;
  return a;
}

static ssa_decode_args base_decode(void) {
  ssa_decode_args a;
  memset(&a, 0, sizeof a);
  a.q = a.out = t4(128, 0);
  a.k_cache = a.v_cache = t4(4096 * 128, 128);
  a.cache_seqlens = (const int32_t*)FAKE;
  a.ssa_n = a.ssa_b = (const float*)FAKE;
  a.workspace = FAKE;
  a.batch = 4, a.heads_q = 8, a.heads_kv = 8, a.capacity = 4096, a.head_dim = 128;
  a.dtype = SSA_DTYPE_BF16, a.softmax_scale = 0.088f;
  return a;
}

typedef int32_t (*bwd_fn)(const ssa_bwd_args*, void*);

/* every integer field of a struct, by offset */
#define INT_FIELDS_FWD {offsetof(ssa_fwd_args, batch), offsetof(ssa_fwd_args, heads_q), \
    offsetof(ssa_fwd_args, heads_kv), offsetof(ssa_fwd_args, seqlen), offsetof(ssa_fwd_args, head_dim), \
    offsetof(ssa_fwd_args, dtype), offsetof(ssa_fwd_args, causal)}
#define INT_FIELDS_BWD {offsetof(ssa_bwd_args, batch), offsetof(ssa_bwd_args, heads_q), \
    offsetof(ssa_bwd_args, heads_kv), offsetof(ssa_bwd_args, seqlen), offsetof(ssa_bwd_args, head_dim), \
    offsetof(ssa_bwd_args, dtype), offsetof(ssa_bwd_args, causal)}
#define INT_FIELDS_DEC {offsetof(ssa_decode_args, batch), offsetof(ssa_decode_args, heads_q), \
    offsetof(ssa_decode_args, heads_kv), offsetof(ssa_decode_args, capacity), \
    offsetof(ssa_decode_args, head_dim), offsetof(ssa_decode_args, dtype), offsetof(ssa_decode_args, num_splits)}

static void set_i32(void* s, size_t off, int32_t v) { memcpy((char*)s + off, &v, sizeof v); }

static void sweep_fwd(void) {
  const size_t f[] = INT_FIELDS_FWD;
  const size_t tens[] = {offsetof(ssa_fwd_args, q), offsetof(ssa_fwd_args, k), offsetof(ssa_fwd_args, v),
                         offsetof(ssa_fwd_args, out)};
  for (int i = 0; i < (int)(sizeof f / sizeof f[0]); ++i)
    for (int j = 0; j < NI; ++j)
      for (int dt = 0; dt < 3; ++dt) {
        ssa_fwd_args a = base_fwd();
        a.dtype = dt;
        set_i32(&a, f[i], kInts[j]);
        ssa_fwd(&a, NULL);
        ssa_varlen_fwd_args va = {a, (const int32_t*)FAKE, kInts[(j + i) % NI]};
        ssa_varlen_fwd(&va, NULL);
        calls += 2;
      }
  for (int i = 0; i < 4; ++i)
    for (int s = 0; s < NS; ++s)
      for (int c = 0; c < 3; ++c) {
        ssa_fwd_args a = base_fwd();
        int64_t* st = (int64_t*)((char*)&a + tens[i] + offsetof(ssa_tensor4, stride_b)) + c;
        *st = kStrides[s];
        ssa_fwd(&a, NULL);
        ++calls;
      }
  expect(ssa_fwd(NULL, NULL), SSA_ERR_NULL_POINTER, "ssa_fwd(NULL)");
  expect(ssa_varlen_fwd(NULL, NULL), SSA_ERR_NULL_POINTER, "ssa_varlen_fwd(NULL)");
  ssa_fwd_args a = base_fwd();
  a.seqlen = INT32_MAX;
  expect(ssa_fwd(&a, NULL), SSA_ERR_SHAPE, "ssa_fwd seqlen INT32_MAX");
  a = base_fwd();
  a.head_dim = 16;
  expect(ssa_fwd(&a, NULL), SSA_ERR_HEAD_DIM, "ssa_fwd bf16 head_dim 16");
  a.dtype = 3;
  expect(ssa_fwd(&a, NULL), SSA_ERR_DTYPE, "ssa_fwd dtype 3");
}

static void sweep_bwd(void) {
  const size_t f[] = INT_FIELDS_BWD;
  const bwd_fn fns[] = {ssa_bwd, ssa_bwd_preprocess, ssa_bwd_dkdv, ssa_bwd_dq, ssa_bwd_reduce, ssa_bwd_noalloc};
  const size_t tens[] = {offsetof(ssa_bwd_args, q), offsetof(ssa_bwd_args, k), offsetof(ssa_bwd_args, v),
                         offsetof(ssa_bwd_args, out), offsetof(ssa_bwd_args, dout), offsetof(ssa_bwd_args, dq),
                         offsetof(ssa_bwd_args, dk), offsetof(ssa_bwd_args, dv)};
  for (int e = 0; e < 6; ++e) {
    for (int i = 0; i < (int)(sizeof f / sizeof f[0]); ++i)
      for (int j = 0; j < NI; ++j)
        for (int dt = 0; dt < 3; ++dt)
          for (int ds = 0; ds < 2; ++ds) {
            ssa_bwd_args a = base_bwd();
            a.dtype = dt;
            a.ds_workspace = ds ? FAKE : NULL;
            set_i32(&a, f[i], kInts[j]);
            fns[e](&a, NULL);
            ++calls;
            if (e == 0) {
              ssa_varlen_bwd_args va = {a, (const int32_t*)FAKE, kInts[(j + i) % NI]};
              ssa_varlen_bwd(&va, NULL);
              ++calls;
            }
          }
    for (int i = 0; i < 8; ++i)
      for (int s = 0; s < NS; ++s)
        for (int c = 0; c < 3; ++c) {
          ssa_bwd_args a = base_bwd();
          int64_t* st = (int64_t*)((char*)&a + tens[i] + offsetof(ssa_tensor4, stride_b)) + c;
          *st = kStrides[s];
          fns[e](&a, NULL);
          ++calls;
        }
    expect(fns[e](NULL, NULL), SSA_ERR_NULL_POINTER, "bwd entry (NULL)");
    ssa_bwd_args a = base_bwd();
    a.heads_kv = 3;
    expect(fns[e](&a, NULL), SSA_ERR_SHAPE, "bwd entry Hq % Hkv");
  }
  expect(ssa_varlen_bwd(NULL, NULL), SSA_ERR_NULL_POINTER, "ssa_varlen_bwd(NULL)");
}

static void sweep_decode(void) {
  const size_t f[] = INT_FIELDS_DEC;
  for (int i = 0; i < (int)(sizeof f / sizeof f[0]); ++i)
    for (int j = 0; j < NI; ++j) {
      ssa_decode_args a = base_decode();
      set_i32(&a, f[i], kInts[j]);
      ssa_decode(&a, NULL);
      ++calls;
    }
  expect(ssa_decode(NULL, NULL), SSA_ERR_NULL_POINTER, "ssa_decode(NULL)");
  ssa_decode_args a = base_decode();
  a.dtype = SSA_DTYPE_FP32;
  expect(ssa_decode(&a, NULL), SSA_ERR_DTYPE, "ssa_decode fp32");
}

static void sweep_queries(void) {
  for (int a = 0; a < NI; ++a)
    for (int b = 0; b < NI; ++b)
      for (int c = 0; c < NI; ++c) {
        const int32_t x = kInts[a], y = kInts[b], z = kInts[c];
        const int64_t r[] = {
            ssa_bwd_partials_count(x, y, z),
            ssa_bwd_ds_workspace_bytes(x, y, z, 1),
            ssa_bwd_ds_workspace_bytes(x, y, z, 0),
            ssa_varlen_bwd_ds_workspace_bytes(x, y, z, x, 1),
            ssa_varlen_bwd_ds_workspace_bytes(x, y, z, z, 0),
            ssa_decode_num_splits(x, y, y, z, 0),
            ssa_decode_num_splits(x, y, z, z, x),
            ssa_decode_workspace_bytes(x, y, y, z, 128, 0),
            ssa_decode_workspace_bytes(x, y, z, y, 64, z),
            ssa_rmsnorm_workspace_floats(x, y),
        };
        for (int i = 0; i < (int)(sizeof r / sizeof r[0]); ++i, ++calls)
          if (r[i] < 0) {
            fprintf(stderr, "FAIL size query %d negative for (%d, %d, %d)\n", i, x, y, z);
            ++failures;
          }
      }
  for (int s = -3; s < 12; ++s)
    if (ssa_status_string(s) == NULL) {
      fprintf(stderr, "FAIL ssa_status_string(%d) is NULL\n", s);
      ++failures;
    }
  expect(ssa_abi_version(), SSA_ABI_VERSION, "ssa_abi_version");
}

static void sweep_decoder_ops(void) {
  for (int j = 0; j < NI; ++j)
    for (int k = 0; k < NI; ++k) {
      ssa_rope_args r = {FAKE, 4096 * 8 * 64, 8 * 64, 64, FAKE, (const float*)FAKE, (const float*)FAKE,
                         4096, 1, 8, 64, 0, 0};
      r.seqlen = kInts[j];
      r.heads = kInts[k];
      ssa_rope(&r, NULL);
      r.seqlen = 4096, r.heads = 8, r.head_dim = kInts[j], r.x_stride_s = kStrides[k % NS];
      ssa_rope(&r, NULL);
      ssa_rmsnorm_fwd_args nf = {FAKE, FAKE, FAKE, (float*)FAKE, kInts[j], kInts[k], 0, 1e-5f};
      ssa_rmsnorm_fwd(&nf, NULL);
      ssa_rmsnorm_bwd_args nb = {FAKE, FAKE, FAKE, (const float*)FAKE, (float*)FAKE, (float*)FAKE,
                                 (float*)FAKE, kInts[j], kInts[k], 0};
      ssa_rmsnorm_bwd(&nb, NULL);
      ssa_swiglu_args sw = {FAKE, FAKE, FAKE, kInts[j], kInts[k], 0, k & 1};
      ssa_swiglu(&sw, NULL);
      ssa_cross_entropy_args ce = {FAKE, FAKE, (float*)FAKE, (float*)FAKE, (const float*)FAKE, FAKE,
                                   kInts[j], kInts[k], 0, k & 1};
      ssa_cross_entropy(&ce, NULL);
      calls += 6;
    }
  expect(ssa_rope(NULL, NULL), SSA_OPS_ERR_NULL_POINTER, "ssa_rope(NULL)");
  expect(ssa_rmsnorm_fwd(NULL, NULL), SSA_OPS_ERR_NULL_POINTER, "ssa_rmsnorm_fwd(NULL)");
  expect(ssa_rmsnorm_bwd(NULL, NULL), SSA_OPS_ERR_NULL_POINTER, "ssa_rmsnorm_bwd(NULL)");
  expect(ssa_swiglu(NULL, NULL), SSA_OPS_ERR_NULL_POINTER, "ssa_swiglu(NULL)");
  expect(ssa_cross_entropy(NULL, NULL), SSA_OPS_ERR_NULL_POINTER, "ssa_cross_entropy(NULL)");
}

int main(void) {
  int devices = 0;
  if (hipGetDeviceCount(&devices) == 0 && devices > 0) {
    printf("skipped: %d GPU(s) visible; this program passes fake device pointers\n", devices);
    return 0;
  }
  sweep_queries();
  sweep_fwd();
  sweep_bwd();
  sweep_decode();
  sweep_decoder_ops();
  printf("host validation: %ld calls, %d failures\n", calls, failures);
  return failures != 0;
}
