/* CPU oracle for the LEMA hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * Nothing in the product (the HIP library and the Python package above it) links, loads or
 * calls this file. Only the tests, the smoke check and the CPU-baseline leg of the benchmark
 * use it, and only as the oracle of the parity checks / the timed CPU counterpart.
 *
 * Each function restates one piece of the reference's behaviour, cited as file:line of
 * moritzbroe/latest_exact_match_attention:
 *
 *   lo_pack_codes          code/lema/attention.py:82-97    bit j of a row's code = (z_j >= 0)
 *   lo_latest_prev_match   verification/lema.py:19-33 and  the dictionary rule: look the query
 *                          code/lema/attention.py:100-132  up, then insert the key
 *   lo_gather              code/lema/attention.py:156-158  y = v[src], miss -> v[0] * 0
 *                          code/lema/csrc/store.cpp:92     (store path: miss -> +0 bytes)
 *   lo_store_exchange      code/lema/csrc/store.cpp:56-162 the shared open-addressing table:
 *                          splitmix64 + fastrange home slot, linear probing, slot layout
 *                          [code u64 | state u64 | value bytes], lookup-then-insert per
 *                          partition in position order, partition-parallel.
 *
 * How each function is pinned (the tests do this): see tests/test_oracle.py.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { LO_F32 = 0, LO_F16 = 1, LO_BF16 = 2 };

/* ------------------------------------------------------------------ scalar conversions */
static float lo_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31;
  const uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ff;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal half: value = man * 2^-24, exact in float */
      float f = (float)man * (1.0f / 16777216.0f);
      memcpy(&bits, &f, 4);
      bits |= sign;
    }
  } else if (exp == 0x1f) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float out;
  memcpy(&out, &bits, 4);
  return out;
}

static float lo_bf16_to_f32(uint16_t b) {
  uint32_t bits = (uint32_t)b << 16;
  float out;
  memcpy(&out, &bits, 4);
  return out;
}

static float lo_load(const void* base, int dtype, int64_t i) {
  switch (dtype) {
    case LO_F32: return ((const float*)base)[i];
    case LO_F16: return lo_f16_to_f32(((const uint16_t*)base)[i]);
    default: return lo_bf16_to_f32(((const uint16_t*)base)[i]);
  }
}

/* ------------------------------------------------------------------------ pack codes */
/* attention.py:95-97: code = sum_j [z_j >= 0] << j. The comparison is a float compare, so
 * -0.0 gives 1 and NaN gives 0. rows are contiguous, D elements each. */
int lo_pack_codes(const void* z, int dtype, int64_t rows, int D, uint64_t* codes) {
  if (D < 1 || D > 64) return 2;
  for (int64_t r = 0; r < rows; ++r) {
    uint64_t c = 0;
    for (int j = 0; j < D; ++j)
      if (lo_load(z, dtype, r * D + j) >= 0.0f) c |= (uint64_t)1 << j;
    codes[r] = c;
  }
  return 0;
}

/* ------------------------------------------------------------ a small code -> pos map */
typedef struct {
  uint64_t* key;
  int64_t* val;
  uint8_t* used;
  uint64_t mask;
} lo_map;

static uint64_t lo_hash(uint64_t x) { /* any decent mixer works for a map */
  x ^= x >> 33;
  x *= 0xff51afd7ed558ccdULL;
  x ^= x >> 33;
  x *= 0xc4ceb9fe1a85ec53ULL;
  x ^= x >> 33;
  return x;
}

static int lo_map_init(lo_map* m, int64_t n) {
  uint64_t size = 16;
  while (size < (uint64_t)(2 * n + 2)) size <<= 1;
  m->key = (uint64_t*)malloc(size * sizeof(uint64_t));
  m->val = (int64_t*)malloc(size * sizeof(int64_t));
  m->used = (uint8_t*)calloc(size, 1);
  m->mask = size - 1;
  return m->key && m->val && m->used ? 0 : -1;
}

static void lo_map_free(lo_map* m) {
  free(m->key);
  free(m->val);
  free(m->used);
}

static int64_t* lo_map_slot(lo_map* m, uint64_t k, int create) {
  uint64_t s = lo_hash(k) & m->mask;
  for (;;) {
    if (!m->used[s]) {
      if (!create) return NULL;
      m->used[s] = 1;
      m->key[s] = k;
      m->val[s] = -1;
      return &m->val[s];
    }
    if (m->key[s] == k) return &m->val[s];
    s = (s + 1) & m->mask;
  }
}

/* ---------------------------------------------------------------- latest prev match */
/* The dictionary rule of verification/lema.py:26-29 on N independent rows of T positions:
 * src[i] = last.get(qc[i], -1); last[kc[i]] = i. Equal to attention.py:100-132's sorted
 * segmented running maximum for every input (strict causality, -1 on a miss). */
int lo_latest_prev_match(const uint64_t* qc, const uint64_t* kc, int64_t N, int64_t T,
                         int64_t* src) {
  if (N < 0 || T < 0) return 2;
  lo_map m;
  if (lo_map_init(&m, T) != 0) return 3;
  for (int64_t n = 0; n < N; ++n) {
    memset(m.used, 0, m.mask + 1);
    const uint64_t* q = qc + n * T;
    const uint64_t* k = kc + n * T;
    int64_t* s = src + n * T;
    for (int64_t i = 0; i < T; ++i) {
      const int64_t* hit = lo_map_slot(&m, q[i], 0);
      s[i] = hit ? *hit : -1;
      *lo_map_slot(&m, k[i], 1) = i;
    }
  }
  lo_map_free(&m);
  return 0;
}

/* ------------------------------------------------------------------------- gather */
/* attention.py:157-158: y = gather(v, src.clamp_min(0)) * (src >= 0), computed in the value
 * dtype. A hit multiplies by 1 (the row's bits, NaN stays NaN); a miss is v[row, 0] * 0,
 * i.e. a zero carrying v[0]'s sign, or NaN where v[0] is inf or NaN. miss_mode 1 is the
 * store path (store.cpp:92): the row is zero bytes. v and y are contiguous [N, T, dv]. */
static uint16_t lo_f32_to_bf16_bits_of_zero_or_nan(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  return (uint16_t)(b >> 16); /* exact for +-0; a quiet NaN keeps a nonzero mantissa */
}

static uint16_t lo_f32_to_f16_bits_of_zero_or_nan(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  const uint16_t sign = (uint16_t)((b >> 16) & 0x8000);
  if ((b & 0x7fffffffu) == 0) return sign;
  return (uint16_t)(sign | 0x7e00u); /* NaN */
}

int lo_gather(const void* v, int dtype, int64_t N, int64_t T, int64_t dv, const int64_t* src,
              int miss_mode, void* y) {
  const int64_t esz = dtype == LO_F32 ? 4 : 2;
  const int64_t rb = dv * esz;
  for (int64_t n = 0; n < N; ++n) {
    const uint8_t* vr = (const uint8_t*)v + n * T * rb;
    uint8_t* yr = (uint8_t*)y + n * T * rb;
    for (int64_t t = 0; t < T; ++t) {
      const int64_t j = src[n * T + t];
      uint8_t* out = yr + t * rb;
      if (j >= 0) {
        if (j >= T) return 2;
        memcpy(out, vr + j * rb, (size_t)rb);
        continue;
      }
      if (miss_mode == 1) {
        memset(out, 0, (size_t)rb);
        continue;
      }
      for (int64_t e = 0; e < dv; ++e) {
        const float x = lo_load(vr, dtype, e) * 0.0f;
        if (dtype == LO_F32) {
          memcpy(out + e * 4, &x, 4);
        } else if (dtype == LO_BF16) {
          uint16_t b = lo_f32_to_bf16_bits_of_zero_or_nan(x);
          memcpy(out + e * 2, &b, 2);
        } else {
          uint16_t b = lo_f32_to_f16_bits_of_zero_or_nan(x);
          memcpy(out + e * 2, &b, 2);
        }
      }
    }
  }
  return 0;
}

/* -------------------------------------------------------------------------- store */
/* The shared table of store.cpp. A slot is [code u64 | state u64 | value bytes] with stride
 * 16 + vbytes; the state word is 0 (free), 1 (being filled) or group + 2 (published). The
 * home slot of (group, code) is Lemire's fastrange of a splitmix64-finalised mix of code and
 * group * 2^64/phi (store.cpp:58-71); probing is linear with wrap-around (store.cpp:80). */
#define LO_EMPTY 0ULL
#define LO_LOCKED 1ULL

static inline uint64_t lo_splitmix_fin(uint64_t x) {
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
  return x ^ (x >> 31);
}

static inline int64_t lo_home(uint64_t code, uint64_t group, int64_t cap) {
  const uint64_t h = lo_splitmix_fin(code ^ (group * 0x9E3779B97F4A7C15ULL));
  return (int64_t)(((unsigned __int128)h * (uint64_t)cap) >> 64);
}

typedef struct {
  uint8_t* base;
  int64_t cap, stride, vbytes;
} lo_table;

static inline uint64_t* lo_code_w(const lo_table* t, int64_t s) {
  return (uint64_t*)(t->base + s * t->stride);
}
static inline uint64_t* lo_state_w(const lo_table* t, int64_t s) {
  return (uint64_t*)(t->base + s * t->stride) + 1;
}
static inline uint8_t* lo_value_p(const lo_table* t, int64_t s) {
  return t->base + s * t->stride + 16;
}

/* store.cpp:84-93: copy the value under (group, code) into dst, or zeros. */
static void lo_read(const lo_table* t, uint64_t c, uint64_t g, uint8_t* dst) {
  const uint64_t tag = g + 2;
  int64_t s = lo_home(c, g, t->cap);
  for (int64_t n = 0; n < t->cap; ++n) {
    const uint64_t st = __atomic_load_n(lo_state_w(t, s), __ATOMIC_ACQUIRE);
    if (st == LO_EMPTY) break;
    if (st == tag && *lo_code_w(t, s) == c) {
      memcpy(dst, lo_value_p(t, s), (size_t)t->vbytes);
      return;
    }
    if (++s == t->cap) s = 0;
  }
  memset(dst, 0, (size_t)t->vbytes);
}

/* store.cpp:97-117: (group, code) -> value, latest wins. 1 = new slot, 0 = overwrite,
 * -1 = every slot probed without finding room (the table is full). */
static int lo_insert(const lo_table* t, uint64_t c, uint64_t g, const uint8_t* src) {
  const uint64_t tag = g + 2;
  int64_t s = lo_home(c, g, t->cap);
  for (int64_t n = 0; n < t->cap; ++n) {
    uint64_t st = __atomic_load_n(lo_state_w(t, s), __ATOMIC_ACQUIRE);
    if (st == LO_EMPTY) {
      uint64_t expect = LO_EMPTY;
      if (__atomic_compare_exchange_n(lo_state_w(t, s), &expect, LO_LOCKED, 0,
                                      __ATOMIC_ACQ_REL, __ATOMIC_ACQUIRE)) {
        *lo_code_w(t, s) = c;
        memcpy(lo_value_p(t, s), src, (size_t)t->vbytes);
        __atomic_store_n(lo_state_w(t, s), tag, __ATOMIC_RELEASE);
        return 1;
      }
      st = expect;
    }
    if (st == tag && *lo_code_w(t, s) == c) {
      memcpy(lo_value_p(t, s), src, (size_t)t->vbytes);
      return 0;
    }
    if (++s == t->cap) s = 0;
  }
  return -1;
}

/* store.cpp:127-162: items i in [0, n) are position i % T of partition i / T (group
 * g0 + i / T); each partition in order: out[i] = lookup(qc[i]), then insert kc[i] -> v[i].
 * added[p] += newly claimed slots. Partitions are split over `nthreads` threads the way
 * at::parallel_for splits them (contiguous blocks, at least max(1, 128 / T) partitions per
 * task, store.cpp:145); prefetch runs 16 items ahead (store.cpp:45, 147-152).
 * Returns 0, or 1 when some insert found the table full (store.cpp:159-160). */
int lo_store_exchange(uint8_t* table, int64_t cap, int64_t vbytes, const uint64_t* qc,
                      const uint64_t* kc, const uint8_t* values, uint8_t* out, int64_t n,
                      int64_t T, int64_t g0, int64_t* added, int nthreads) {
  if (T <= 0 || n % T != 0 || cap <= 0 || vbytes <= 0 || vbytes % 8 != 0) return 2;
  const int64_t P = n / T;
  lo_table tb = {table, cap, 16 + vbytes, vbytes};
  int full = 0;
  const int64_t grain = 128 / T > 1 ? 128 / T : 1;
  int64_t tasks = (P + grain - 1) / grain;
  if (nthreads < 1) nthreads = 1;
  if (tasks > nthreads) tasks = nthreads;
  if (tasks < 1) tasks = 1;
  const int64_t per = (P + tasks - 1) / tasks;
#pragma omp parallel for num_threads((int)tasks) schedule(static, 1) reduction(| : full)
  for (int64_t task = 0; task < tasks; ++task) {
    const int64_t p_lo = task * per;
    const int64_t p_hi = p_lo + per < P ? p_lo + per : P;
    if (p_lo >= p_hi) continue;
    const int64_t lo = p_lo * T, hi = p_hi * T;
    for (int64_t i = lo; i < lo + 16 && i < hi; ++i) {
      __builtin_prefetch(tb.base + lo_home(qc[i], (uint64_t)(g0 + i / T), cap) * tb.stride);
      __builtin_prefetch(tb.base + lo_home(kc[i], (uint64_t)(g0 + i / T), cap) * tb.stride);
    }
    for (int64_t i = lo; i < hi; ++i) {
      if (i + 16 < hi) {
        const uint64_t ga = (uint64_t)(g0 + (i + 16) / T);
        __builtin_prefetch(tb.base + lo_home(qc[i + 16], ga, cap) * tb.stride);
        __builtin_prefetch(tb.base + lo_home(kc[i + 16], ga, cap) * tb.stride);
      }
      const uint64_t g = (uint64_t)(g0 + i / T);
      lo_read(&tb, qc[i], g, out + i * vbytes);
      const int r = lo_insert(&tb, kc[i], g, values + i * vbytes);
      if (r < 0)
        full = 1;
      else
        added[i / T] += r;
    }
  }
  return full ? 1 : 0;
}

/* The home slot, exported so tests can place keys deliberately (collisions, wrap-around). */
int64_t lo_store_home(uint64_t code, uint64_t group, int64_t cap) {
  return lo_home(code, group, cap);
}

int lo_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
