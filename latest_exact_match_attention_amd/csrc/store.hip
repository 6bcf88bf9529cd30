// The LEMA retrieval store in HBM: one open-addressing table shared by every (layer, stream,
// head) partition, replacing the reference's host-RAM store (code/lema/csrc/store.cpp,
// driven by code/lema/cache.py:129-302).
//
// Table format -- identical to the reference's, so a table is interchangeable byte for byte:
// slot s is [code u64 | state u64 | value bytes] at s * (16 + vbytes); state 0 = free,
// group + 2 = taken (the reference also passes through 1 while a slot is filled; no completed
// exchange leaves it, and this store never writes it). The home slot of (group, code) is Lemire's fastrange of
// the splitmix64 finaliser of code ^ (group * 2^64/phi) (store.cpp:58-71); probing is linear with
// wrap-around. A zeroed allocation is an empty table.
//
// Exchange semantics (store.cpp:122-162): items i in [0, n) are position i % T of partition
// i / T, group g0 + i / T; in position order within a partition each item looks its query code
// up (value, or zeros) and then inserts its key code -> value (latest write wins); counts[g]
// grows by the newly claimed slots; a key that finds no free slot sets *full.
//
// GPU execution. Partitions run concurrently; the only cross-partition interaction is slot
// claiming: a device-scope CAS of the state word from free straight to the claimer's tag, then
// plain stores of code and value. No reader in the same kernel ever reads a slot it did not
// find before the kernel started -- another partition's slot is skipped on its tag, and a
// partition's own new slots are only probed for "free" -- so the claim needs no intermediate
// state and no fence; the kernel boundary publishes code and value to later exchanges. Every
// slot in front of an entry on its probe path was occupied before the entry was made, so a
// stale read can only show a free slot where someone is claiming: header reads are hints, the
// CAS decides.
//   * T == 1 (a decode step): one kernel; 8 lanes per item read the query's and the key's
//     first 8-slot windows together (one ballot each), look the query up, then update the
//     key's entry or claim a slot for it.
//   * T >= 2: sub-chunks of up to 1024 positions, one launch per sub-chunk (in order), one
//     workgroup per partition: in-chunk matches come from the LDS resolver, other queries from
//     the table; after a workgroup barrier (no query may see a later key) each key code's
//     last occurrence overwrites its existing entry, and after another barrier the codes that
//     had none claim new slots.
#include "resolve_core.h"

namespace lema {
namespace {

constexpr uint64_t kStateEmpty = 0;
// Lanes probing one item together: one window of kGroup slots per round trip.
#ifndef LEMA_STORE_GROUP
#define LEMA_STORE_GROUP 8
#endif
constexpr int kGroup = LEMA_STORE_GROUP;
static_assert(kGroup == 4 || kGroup == 8 || kGroup == 16 || kGroup == 32, "probe group width");

__device__ __forceinline__ uint64_t splitmix_fin(uint64_t x) {
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

__device__ __forceinline__ int64_t home_slot(uint64_t code, uint64_t group, int64_t cap) {
  const uint64_t h = splitmix_fin(code ^ (group * 0x9E3779B97F4A7C15ull));
  return static_cast<int64_t>(__umul64hi(h, static_cast<uint64_t>(cap)));
}

struct StoreArgs {
  uint8_t* table;
  int64_t cap, stride, vbytes;
  const void* qc;  // null: insert only
  const void* kc;
  int32_t code_bytes;
  const uint8_t* values;
  uint8_t* out;  // null when qc is null
  int64_t n, T, g0;
  int64_t s0;   // first position of the sub-chunk (T >= 2)
  int32_t len;  // positions in the sub-chunk
  int32_t piece;  // 16 or 8: value bytes copied per lane
  unsigned long long* counts;
  int32_t* full;
};

__device__ __forceinline__ uint64_t code_at(const void* base, int32_t cb, int64_t i) {
  return cb == 4 ? static_cast<uint64_t>(static_cast<const uint32_t*>(base)[i])
                 : static_cast<const uint64_t*>(base)[i];
}

__device__ __forceinline__ uint64_t* state_ptr(const StoreArgs& a, int64_t s) {
  return reinterpret_cast<uint64_t*>(a.table + s * a.stride) + 1;
}

// Copy one value row with the group's lanes (src null: write zeros).
__device__ __forceinline__ void group_copy(const StoreArgs& a, uint8_t* dst, const uint8_t* src,
                                           int gl) {
  const int pieces = static_cast<int>(a.vbytes / a.piece);
  for (int k = gl; k < pieces; k += kGroup) {
    if (a.piece == 16) {
      const u32x4 v = src ? *reinterpret_cast<const u32x4*>(src + 16 * k) : u32x4{0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4*>(dst + 16 * k) = v;
    } else {
      const u32x2 v = src ? *reinterpret_cast<const u32x2*>(src + 8 * k) : u32x2{0u, 0u};
      *reinterpret_cast<u32x2*>(dst + 8 * k) = v;
    }
  }
}

// The window of kGroup slots starting at `base` (wrapping); lane gl reads slot base + gl.
// Lanes beyond the `left` slots still to probe report nothing. Returns this group's bits.
struct Window {
  uint32_t match, empty;
};
__device__ __forceinline__ Window read_window(const StoreArgs& a, int64_t base, int64_t left,
                                              uint64_t code, uint64_t tag, int gl, int gbase) {
  bool m = false, e = false;
  if (gl < left) {
    int64_t s = base + gl;
    if (s >= a.cap) s -= a.cap;
    const uint64_t* hdr = reinterpret_cast<const uint64_t*>(a.table + s * a.stride);
    const uint64_t st = hdr[1];
    m = st == tag && hdr[0] == code;
    e = st == kStateEmpty;
  }
  const uint64_t mask = kGroup == 64 ? ~0ull : ((1ull << kGroup) - 1);
  return Window{static_cast<uint32_t>((__ballot(m) >> gbase) & mask),
                static_cast<uint32_t>((__ballot(e) >> gbase) & mask)};
}

// Slot of (tag, code) or -1 (code/lema/csrc/store.cpp:84-93), starting from the first window
// w0 read at `base` = home. Group-uniform.
__device__ int64_t group_lookup(const StoreArgs& a, uint64_t code, uint64_t tag, int64_t base,
                                Window w0, int gl, int gbase) {
  for (int64_t left = a.cap; left > 0; left -= kGroup) {
    const Window w = left == a.cap ? w0 : read_window(a, base, left, code, tag, gl, gbase);
    const int fm = w.match ? __ffs(w.match) - 1 : kGroup;
    const int fe = w.empty ? __ffs(w.empty) - 1 : kGroup;
    if (fm < fe) {
      const int64_t s = base + fm;
      return s >= a.cap ? s - a.cap : s;
    }
    if (w.empty) return -1;
    base += kGroup;
    if (base >= a.cap) base -= a.cap;
  }
  return -1;
}

// Insert (tag, code) -> value (code/lema/csrc/store.cpp:97-117), starting from the first
// window w0 read at `base` = home: 1 = claimed a new slot, 0 = overwrote the partition's own
// entry, -1 = probed every slot without room. With `claim_only` the key is known to be absent
// and only free slots are looked for. Group-uniform.
__device__ int group_insert(const StoreArgs& a, uint64_t code, uint64_t tag, const uint8_t* value,
                            int64_t base, Window w0, bool claim_only, int gl, int gbase) {
  for (int64_t left = a.cap; left > 0; left -= kGroup) {
    const Window w = left == a.cap ? w0 : read_window(a, base, left, code, tag, gl, gbase);
    const int fm = (!claim_only && w.match) ? __ffs(w.match) - 1 : kGroup;
    uint32_t empty = w.empty;
    if (fm < kGroup && (!empty || fm < __ffs(empty) - 1)) {
      int64_t s = base + fm;
      if (s >= a.cap) s -= a.cap;
      group_copy(a, a.table + s * a.stride + 16, value, gl);
      return 0;
    }
    while (empty) {  // claim the first free slot; a lost race just marks that slot taken
      const int e = __ffs(empty) - 1;
      int64_t s = base + e;
      if (s >= a.cap) s -= a.cap;
      unsigned long long old = 0;
      if (gl == e)
        old = atomicCAS(reinterpret_cast<unsigned long long*>(state_ptr(a, s)), kStateEmpty, tag);
      const bool won = __shfl(old == kStateEmpty ? 1 : 0, gbase + e) != 0;
      if (won) {
        if (gl == e) *reinterpret_cast<uint64_t*>(a.table + s * a.stride) = code;
        group_copy(a, a.table + s * a.stride + 16, value, gl);
        return 1;
      }
      empty &= ~(1u << e);
    }
    base += kGroup;
    if (base >= a.cap) base -= a.cap;
  }
  return -1;
}

// A decode step (T == 1): item i is partition i; 8 lanes per item.
__global__ __launch_bounds__(256) void store_step_kernel(StoreArgs a) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t i = gid / kGroup;
  const int lane = threadIdx.x & 63, gl = lane % kGroup, gbase = lane - gl;
  if (i >= a.n) return;  // whole groups only: n is a count of items, groups are aligned
  const uint64_t tag = static_cast<uint64_t>(a.g0 + i) + 2;
  const uint64_t kcode = code_at(a.kc, a.code_bytes, i);
  const int64_t khome = home_slot(kcode, tag - 2, a.cap);
  const uint64_t qcode = a.qc != nullptr ? code_at(a.qc, a.code_bytes, i) : 0;
  const int64_t qhome = a.qc != nullptr ? home_slot(qcode, tag - 2, a.cap) : 0;
  // the two first windows are independent: both reads are in flight together
  const Window wk = read_window(a, khome, a.cap, kcode, tag, gl, gbase);
  const Window wq = a.qc != nullptr ? read_window(a, qhome, a.cap, qcode, tag, gl, gbase)
                                    : Window{0u, 0u};
  if (a.qc != nullptr) {
    const int64_t s = group_lookup(a, qcode, tag, qhome, wq, gl, gbase);
    group_copy(a, a.out + i * a.vbytes, s >= 0 ? a.table + s * a.stride + 16 : nullptr, gl);
  }
  const int r = group_insert(a, kcode, tag, a.values + i * a.vbytes, khome, wk, false, gl, gbase);
  if (gl == 0) {
    if (r > 0) atomicAdd(&a.counts[a.g0 + i], 1ull);
    if (r < 0) atomicOr(a.full, 1);
  }
}

// One sub-chunk [s0, s0 + len) of every partition, one workgroup (256 threads) per partition.
template <typename CodeT>
__global__ __launch_bounds__(kThreads) void store_chunk_kernel(StoreArgs a) {
  __shared__ ResolveLds<CodeT> s;
  __shared__ int32_t src_in[kChunk];
  __shared__ uint8_t klast[kChunk];
  const int64_t p = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, gl = lane % kGroup, gbase = lane - gl;
  const int grp = t / kGroup;
  constexpr int kGroups = kThreads / kGroup;
  const int64_t first = p * a.T + a.s0;  // item index of the sub-chunk's position 0
  const uint64_t tag = static_cast<uint64_t>(a.g0 + p) + 2;
  const int n = a.len;
  const CodeT SENT = sentinel<CodeT>();

  // 1. queries answered inside the sub-chunk (latest earlier key with the same code)
  if (a.qc != nullptr) {
    ResolveArgs ra{};
    ra.qc = static_cast<const CodeT*>(a.qc) + first;
    ra.kc = static_cast<const CodeT*>(a.kc) + first;
    ra.N = 1;
    ra.T = n;
    ra.nchunks = 1;
    ra.kvec = 0;
    ra.src = nullptr;
    int32_t src[kPer];
    resolve_chunk(s, ra, 0, 0, t, [] { __syncthreads(); }, src);
#pragma unroll
    for (int q = 0; q < kPer; ++q) src_in[q * kThreads + t] = src[q];
  }
  __syncthreads();

  // 2. the last occurrence of every key code in the sub-chunk (latest wins on insert)
  const CodeT* kr = static_cast<const CodeT*>(a.kc) + first;
  for (int x = t; x < kSlots; x += kThreads) s.code[x] = SENT;
  for (int x = t; x <= kSlots; x += kThreads) s.pos[x] = -1;
  __syncthreads();
  int ks[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int o = q * kThreads + t;
    ks[q] = kSlots;
    if (o >= n) continue;
    const CodeT c = kr[o];
    if (c != SENT) {
      bool ins;
      ks[q] = table_claim<CodeT, kBuckets>(s.code, c, SENT, bucket_of<kBuckets>(fold(c)), ins);
    }
    atomicMax(&s.pos[ks[q]], o);
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int o = q * kThreads + t;
    if (o < n) klast[o] = s.pos[ks[q]] == o ? 1 : 0;
  }
  __syncthreads();

  // 3. look the queries up: in-chunk matches copy the sub-chunk's own values
  if (a.qc != nullptr) {
    for (int o = grp; o < n; o += kGroups) {
      const int j = src_in[o];
      uint8_t* dst = a.out + (first + o) * a.vbytes;
      if (j >= 0) {
        group_copy(a, dst, a.values + (first + j) * a.vbytes, gl);
      } else {
        const uint64_t c = code_at(a.qc, a.code_bytes, first + o);
        const int64_t h = home_slot(c, tag - 2, a.cap);
        const int64_t sl = group_lookup(a, c, tag, h, read_window(a, h, a.cap, c, tag, gl, gbase),
                                        gl, gbase);
        group_copy(a, dst, sl >= 0 ? a.table + sl * a.stride + 16 : nullptr, gl);
      }
    }
  }
  __syncthreads();  // every query of this partition has read the table before any insert

  // 4. each key code's last occurrence overwrites its existing entry; codes without one are
  // marked (klast = 2) and, once no sibling can still be looking entries up, claim a slot
  for (int o = grp; o < n; o += kGroups) {
    if (!klast[o]) continue;
    const uint64_t c = code_at(a.kc, a.code_bytes, first + o);
    const int64_t h = home_slot(c, tag - 2, a.cap);
    const int64_t sl = group_lookup(a, c, tag, h, read_window(a, h, a.cap, c, tag, gl, gbase),
                                    gl, gbase);
    if (sl >= 0)
      group_copy(a, a.table + sl * a.stride + 16, a.values + (first + o) * a.vbytes, gl);
    else if (gl == 0)
      klast[o] = 2;
  }
  __syncthreads();
  int added = 0;
  for (int o = grp; o < n; o += kGroups) {
    if (klast[o] != 2) continue;
    const uint64_t c = code_at(a.kc, a.code_bytes, first + o);
    const int64_t h = home_slot(c, tag - 2, a.cap);
    const int r = group_insert(a, c, tag, a.values + (first + o) * a.vbytes, h,
                               read_window(a, h, a.cap, c, tag, gl, gbase), true, gl, gbase);
    if (r > 0) ++added;
    if (r < 0 && gl == 0) atomicOr(a.full, 1);
  }
  if (gl == 0 && added > 0) atomicAdd(&a.counts[a.g0 + p], static_cast<unsigned long long>(added));
}

}  // namespace
}  // namespace lema

using namespace lema;

extern "C" int lema_store_exchange(void* table, int64_t cap, int64_t vbytes, const void* qc,
                                   const void* kc, int32_t code_bytes, const void* values,
                                   void* out, int64_t n, int64_t T, int64_t g0, int64_t* counts,
                                   int32_t* full, void* stream) {
  clear_error();
  LEMA_REQUIRE(cap >= 1, "capacity must be positive, got %lld", (long long)cap);
  LEMA_REQUIRE(vbytes > 0 && vbytes % 8 == 0,
               "value row of %lld bytes breaks slot alignment (must be a multiple of 8)",
               (long long)vbytes);
  LEMA_REQUIRE(code_bytes == 4 || code_bytes == 8, "code_bytes must be 4 or 8, got %d", code_bytes);
  LEMA_REQUIRE(T > 0 && n >= 0 && n % T == 0, "items must be partitions x T (n=%lld, T=%lld)",
               (long long)n, (long long)T);
  LEMA_REQUIRE(g0 >= 0, "negative group offset");
  if (n == 0) return LEMA_OK;
  LEMA_REQUIRE(table != nullptr && kc != nullptr && values != nullptr && counts != nullptr &&
                   full != nullptr, "null pointer");
  LEMA_REQUIRE(qc == nullptr || out != nullptr, "queries need an output buffer");
  LEMA_REQUIRE(aligned(table, 8) && aligned(kc, code_bytes) && aligned(values, 8) &&
                   aligned(counts, 8) && aligned(full, 4) &&
                   (qc == nullptr || (aligned(qc, code_bytes) && aligned(out, 8))),
               "misaligned pointer");
  StoreArgs a{};
  a.table = static_cast<uint8_t*>(table);
  a.cap = cap;
  a.stride = 16 + vbytes;
  a.vbytes = vbytes;
  a.qc = qc;
  a.kc = kc;
  a.code_bytes = code_bytes;
  a.values = static_cast<const uint8_t*>(values);
  a.out = static_cast<uint8_t*>(out);
  a.n = n;
  a.T = T;
  a.g0 = g0;
  a.counts = reinterpret_cast<unsigned long long*>(counts);
  a.full = full;
  const bool p16 = vbytes % 16 == 0 && aligned(table, 16) && aligned(values, 16) &&
                   (out == nullptr || aligned(out, 16));
  a.piece = p16 ? 16 : 8;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t P = n / T;
  if (T == 1) {
    const int64_t threads = n * kGroup;
    const int64_t grid = (threads + 255) / 256;
    LEMA_REQUIRE(grid < (int64_t(1) << 31), "too many items (%lld)", (long long)n);
    store_step_kernel<<<dim3(grid), dim3(256), 0, st>>>(a);
    return launch_status("store_step_kernel");
  }
  LEMA_REQUIRE(P < (int64_t(1) << 31), "too many partitions (%lld)", (long long)P);
  for (int64_t s0 = 0; s0 < T; s0 += kChunk) {
    a.s0 = s0;
    a.len = static_cast<int32_t>(T - s0 < kChunk ? T - s0 : kChunk);
    if (code_bytes == 4)
      store_chunk_kernel<uint32_t><<<dim3(P), dim3(kThreads), 0, st>>>(a);
    else
      store_chunk_kernel<uint64_t><<<dim3(P), dim3(kThreads), 0, st>>>(a);
    if (int rc = launch_status("store_chunk_kernel")) return rc;
  }
  return LEMA_OK;
}
