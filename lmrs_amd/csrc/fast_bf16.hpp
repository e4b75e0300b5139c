// fast_bf16.hpp -- the bf16 sampling kernel for rows of up to kFastMaxVocab.
//
// One workgroup of 512 threads (one per CU at this LDS size; 8 waves, so each
// thread may hold 256 VGPRs) owns one row.  Its waves are specialised: wave 0
// handles the history (below) while waves 1..7, the row threads, stream the
// row.  Each row thread loads its NCH 16-byte chunks (chunk c = s * 448 + row
// thread) in one burst at kernel entry and converts them to 16-bit
// total-order keys of the RAW logits;
// that single pass over registers also records, in LDS, the largest
// non-history key of every chunk (the "chunk maxima", 2 bytes per 8 logits).
// After it the row's registers are dead on the top-k and greedy paths: every
// later step is a short loop over LDS data (chunk maxima, the history
// members, candidate lists) plus a re-read of the few chunks whose maximum
// can hold a candidate.  Keeping the code after the load pass small matters
// as much as its arithmetic: each row executes it once, so its instructions
// are fetched cold.
//
// Penalties never touch the per-element pass.  The history wave loads the
// history ids, finds the distinct tokens ("members", at most kFastMembers)
// with an LDS hash, fetches their raw logits with one load each and computes
// their penalised keys z (Repetition then Presence/Frequency, bf16-rounded
// per op, as the reference's chain of kernels), all while the row streams in.  Chunk maxima
// skip members; members take part in every selection through their z keys.
// Temperature is not applied per element either: y = bf16(fma(z, 1/T, 0)) is
// monotone in z, so selection runs on z keys and maps only the keys that
// matter to y; runs of z keys that round to one y form one tie group, whose
// tokens are ordered by index as the reference's sort orders them.
//
// Paths after the load pass:
//   greedy   (top_k == 1): the largest z is the largest chunk maximum or
//            member key; the lowest index of its tie group comes from the
//            chunks whose maximum reaches the group.
//   small k  (top_k <= kGatherCap): the k-th largest value among chunk maxima
//            and member keys, L, bounds the k-th largest z from below (each
//            value is a distinct element).  Every element with z at or above
//            the start of L's tie group is gathered (re-reading the chunks
//            whose maximum reaches it), sorted exactly -- inside one wave
//            when there are at most 64 -- and finished in f64.
//   full     (otherwise): a 65536-bin count histogram of the keys in
//            registers (two 16-bit counters per LDS word), compacted to its
//            non-empty keys; per-key weights exp(f64(y - max)) times counts
//            give exact cumulative masses for the top-k cut, the nucleus cut
//            and the draw; the chosen token is the j-th lowest index of its
//            tie group, found on a second read of the row.
// Rows this kernel does not take (a NaN anywhere, more than kFastMembers
// distinct history tokens, a histogram count above 65535, more than
// kMaxEntries distinct keys, more candidates than the lists hold) go through
// the generic engine inside the same workgroup.
#pragma once

#include "generic_engine.hpp"

namespace lmrs {

constexpr int kFT = 512;            // threads of a fast-kernel workgroup
constexpr int kFW = kFT / 64;       // its waves
constexpr int kHW = 0;              // leading waves that hold no row data
constexpr int kRT = kFT - 64 * kHW; // row threads
constexpr int kRW = kRT / 64;       // row waves
constexpr int kMaxEntries = 6144;   // distinct keys the full path keeps in LDS
constexpr int kFastMembers = 2048;  // distinct history tokens the fast path keeps
constexpr int kMaxSlots = 40;       // chunk slots per row thread
constexpr int kFastMaxVocab = kMaxSlots * 8 * kRT;
constexpr int kMaxWindow = kFT;     // widest window of the count cascade (one bin per thread)
constexpr int kHistPer = LMRS_MAX_HISTORY / kFT;
constexpr int kMemPer = kFastMembers / kFT;

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Loads of the row and of the history ids are issued through inline assembly
// and waited for explicitly.  Written as ordinary loads, the compiler moves
// each one down to its first use, after the history work, so that the row
// stream would only start once that work is done; and its own wait for the
// history ids would count the row's loads issued before them.  The waits
// below count loads issued after the one waited for; compiler-issued vector
// memory operations in between only make them wait longer, never shorter.
__device__ __forceinline__ u32x4 issue_load_b128(const void *p) {
  u32x4 d;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(d) : "v"(p));
  return d;
}

__device__ __forceinline__ uint32_t issue_load_b32(const void *p) {
  uint32_t d;
  asm volatile("global_load_dword %0, %1, off" : "=v"(d) : "v"(p));
  return d;
}

__device__ __forceinline__ uint32_t issue_load_u16(const void *p) {
  uint32_t d;
  asm volatile("global_load_ushort %0, %1, off" : "=v"(d) : "v"(p));
  return d;
}

// Calls f(std::integral_constant<int, I>) for I = B .. E-1, each with a
// compile-time index.
template <int I>
struct Index {
  static constexpr int value = I;
};
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (B < E) {
    f(Index<B>{});
    static_for<B + 1, E>(f);
  }
}

// A pointer the compiler must treat as freshly computed: address arithmetic
// of later passes is then not merged with the load phase's, whose results
// would otherwise stay live (and spill) in between.
template <class T>
__device__ __forceinline__ const T *fresh(const T *p) {
  asm volatile("" : "+v"(p));
  return p;
}

__device__ __forceinline__ int fresh_tid() {
  int t = (int)threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// Waits until at most N vector memory operations are outstanding; `d`, the
// destination of an earlier issue_load, is valid afterwards.
template <int N>
__device__ __forceinline__ void wait_loads(u32x4 &d) {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%1)" : "+v"(d) : "n"(N));
}

template <int N>
__device__ __forceinline__ void wait_loads(uint32_t &d) {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%1)" : "+v"(d) : "n"(N));
}


// Padding of a row's last chunk slot: eight bf16 -inf, whose key (0x007F) is
// the lowest non-NaN key.  Counts at that key are corrected for the padding.
__device__ const uint4 kNegInfChunk = {0xFF80FF80u, 0xFF80FF80u, 0xFF80FF80u, 0xFF80FF80u};
constexpr uint32_t kNegInfKey16 = 0x007Fu;

__device__ __forceinline__ uint32_t pk_max_u16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, a),
                                                                __builtin_bit_cast(u16x2, b)));
}

__device__ __forceinline__ uint32_t pk_min_u16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(u16x2, a),
                                                                __builtin_bit_cast(u16x2, b)));
}

// Order keys of two packed bf16 values: flip all bits of negatives, set the
// sign bit of non-negatives (per 16-bit half).
__device__ __forceinline__ uint32_t key_pair(uint32_t w) {
  const uint32_t sgn = (w >> 15) & 0x00010001u;
  return w ^ (sgn * 0x7FFFu + 0x80008000u);
}

__device__ __forceinline__ uint32_t key16_bits(uint32_t k) {
  return (k & 0x8000u) ? (k & 0x7FFFu) : (~k & 0xFFFFu);
}

__device__ __forceinline__ uint32_t bits_key16(uint32_t b) {
  return (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
}

// The temperature processor as a map on 16-bit keys (z -> y).
__device__ __forceinline__ uint32_t temp_key16(uint32_t zk, const RowCfg &c) {
  if (!c.temp_on) return zk;
  const uint32_t yb = f32_to_bf16_dev(__builtin_fmaf(bf16_to_f32(key16_bits(zk)), c.scale, 0.0f));
  return bits_key16(yb);
}

__device__ __forceinline__ float key16_value(uint32_t k) { return bf16_to_f32(key16_bits(k)); }

__device__ __forceinline__ bool is_nan_key16(uint32_t k) { return k >= 0xFF81u || k <= 0x007Eu; }

// Largest of the eight 16-bit keys packed in one chunk.
__device__ __forceinline__ uint32_t chunk_max(const uint32_t (&w)[4]) {
  const uint32_t m = pk_max_u16(pk_max_u16(w[0], w[1]), pk_max_u16(w[2], w[3]));
  return max(m & 0xFFFFu, m >> 16);
}

// Key e (0..7) of a chunk of four packed words, e not known at compile time:
// a select between two 64-bit halves and a shift (an indexed read of the
// four words would be placed in scratch memory).
__device__ __forceinline__ uint32_t chunk_key(const uint4 &w, uint32_t e) {
  const uint64_t lo = ((uint64_t)w.y << 32) | w.x, hi = ((uint64_t)w.w << 32) | w.z;
  const uint64_t v = (e & 4u) ? hi : lo;
  return (uint32_t)(v >> ((e & 3u) * 16u)) & 0xFFFFu;
}

// The lowest z key of the tie group (equal y under temperature) of key z.
__device__ __forceinline__ uint32_t group_low(uint32_t z, const RowCfg &c) {
  if (!c.temp_on) return z;
  const uint32_t y = temp_key16(z, c);
  while (z > 0u && temp_key16(z - 1u, c) == y) --z;
  return z;
}

// Repetition then Presence/Frequency on one history token (bf16 pattern in
// and out), rounding to bf16 after every op (repetition.rs:113-116,
// presence.rs:114-129).
__device__ __forceinline__ uint32_t penalise_member(uint32_t raw, uint32_t count, const RowCfg &c) {
  float v = bf16_to_f32(raw);
  if (c.rep_on) {
    const float pos = round_bf16_dev(v * c.pf), neg = round_bf16_dev(v * c.nf);
    v = (v >= 0.0f) ? pos : neg;
  }
  if (c.pres_on) v = round_bf16_dev(v - round_bf16_host(c.presence + c.frequency * (float)count));
  return __float_as_uint(v) >> 16;
}

// LDS arena with phase-dependent views (byte offsets):
//   [0, 64K)      history hash: token + 1, multiplicity | raw key << 16
//                 (history build); then SelState [0, 57K): gather list, sort
//                 and finish scratch
//                 [60K, 64K): window histogram of the count cascade
//   [64K, 84K)    membership bitmap over the vocab
//   [136K, 152K)  member list: token ids, raw key | z key << 16
//   full path: [0, 128K) 65536 16-bit counters; after compaction [128K, 152K)
//   the entries (key << 16 | count) and [0, 72K) their prefixes; for the
//   final search the member list is rebuilt and [128K, 134K) holds the
//   per-slot / per-thread counts of the ordered search
constexpr int kArenaBytes = 152 * 1024;
constexpr int kOffBitmap = 64 * 1024;
constexpr int kOffWhist = 60 * 1024;
constexpr int kOffSlotCnt = 128 * 1024;
constexpr int kOffTcnt = kOffSlotCnt + kMaxSlots * kRW * 4;
constexpr int kOffMembers = 136 * 1024;
constexpr int kOffEntries = 128 * 1024;
static_assert((int)sizeof(SelState) <= kOffBitmap, "SelState view");
static_assert(kOffBitmap + (kFastMaxVocab + 31) / 32 * 4 <= kOffSlotCnt, "bitmap view");
static_assert((int)sizeof(SelState) <= kOffWhist && kOffWhist + kMaxWindow * 4 <= kOffBitmap, "window view");
static_assert(kOffTcnt + kRT * 4 <= kOffMembers, "count views");
static_assert(kOffMembers + kFastMembers * 8 <= kArenaBytes, "member view");
static_assert(kOffEntries + kMaxEntries * 4 <= kArenaBytes, "entries view");
static_assert(kMaxEntries * 12 <= kOffEntries, "prefix view");
static_assert(kFastMembers % kFT == 0 && LMRS_MAX_HISTORY % kFT == 0, "per-thread counts");

struct FastShared {
  alignas(16) unsigned char arena[kArenaBytes];
  double dscr[kWaves];
  uint32_t uscr[kWaves];
  uint32_t uscr2[kWaves];
  int32_t iscr[kWaves];
  uint32_t chunk_z[8];
  uint32_t bsel[8];

  __device__ uint32_t *u32(int off) { return (uint32_t *)(arena + off); }
  __device__ uint32_t *m_idx() { return u32(kOffMembers); }
  __device__ uint32_t *m_key() { return u32(kOffMembers + kFastMembers * 4); }
  __device__ uint32_t *bitmap() { return u32(kOffBitmap); }
  __device__ uint32_t *whist() { return u32(kOffWhist); }
  __device__ SelState &ss() { return *(SelState *)(arena); }
};

// The fast and the generic engine share one LDS allocation.
union FastOrGeneric {
  FastShared f;
  GenericShared g;
};

__device__ __forceinline__ bool member_bit(const uint32_t *bitmap, uint32_t i) {
  return (bitmap[i >> 5] >> (i & 31u)) & 1u;
}

// Two block-wide maxima with one pair of barriers.
__device__ __forceinline__ void block_max2(uint32_t &a, uint32_t &b, FastShared &sh) {
  a = wave_max(a);
  b = wave_max(b);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    sh.uscr[threadIdx.x >> 6] = a;
    sh.uscr2[threadIdx.x >> 6] = b;
  }
  __syncthreads();
  uint32_t ra = sh.uscr[0], rb = sh.uscr2[0];
#pragma unroll
  for (int i = 1; i < kFW; ++i) {
    ra = max(ra, sh.uscr[i]);
    rb = max(rb, sh.uscr2[i]);
  }
  a = uniform(ra);
  b = uniform(rb);
}

// ---- history members ------------------------------------------------------------

// History tables of the row in LDS: hash (token + 1 -> multiplicity) and the
// membership bitmap; `hid` holds this thread's history ids (strided by the
// block; entries at or past h_len are ignored).  Ends with a barrier.
__device__ __forceinline__ void insert_history(FastShared &sh, const uint32_t (&hid)[kHistPer], int64_t h_len,
                                               int64_t V) {
  uint32_t *hkeys = sh.u32(0), *hcnt = sh.u32(kHashCap * 4), *bitmap = sh.bitmap();
  // First probes of all this thread's ids together (independent atomics in
  // flight at once); the few that collide continue probing afterwards.
  uint32_t sl[kHistPer], prev[kHistPer];
  bool live[kHistPer];
#pragma unroll
  for (int q = 0; q < kHistPer; ++q) {
    const uint32_t t = hid[q];
    live[q] = (int64_t)threadIdx.x + (int64_t)q * kFT < h_len && (int64_t)t < V;
    sl[q] = hash_slot(t);
    prev[q] = 0u;
    if (live[q]) {
      atomicOr(&bitmap[t >> 5], 1u << (t & 31u));
      prev[q] = atomicCAS(&hkeys[sl[q]], 0u, t + 1u);
    }
  }
#pragma unroll
  for (int q = 0; q < kHistPer; ++q) {
    if (live[q]) {
      const uint32_t t = hid[q];
      uint32_t p = prev[q], s2 = sl[q];
      while (p != 0u && p != t + 1u) {  // terminates: the table is at most half full
        s2 = (s2 + 1u) & (kHashCap - 1);
        p = atomicCAS(&hkeys[s2], 0u, t + 1u);
      }
      atomicAdd(&hcnt[s2], 1u);
    }
  }
  __syncthreads();
}

// Clears the hash and the bitmap.  Ends with a barrier.
__device__ __forceinline__ void clear_history(FastShared &sh) {
  uint4 *p = (uint4 *)sh.u32(0);
  constexpr int kVec = (kOffBitmap + kFastMaxVocab / 8) / 16;
  for (int i = threadIdx.x; i < kVec; i += kFT) p[i] = make_uint4(0u, 0u, 0u, 0u);
  __syncthreads();
}

// Compacts the hash into the member list (token ids; multiplicities in
// m_key until the keys replace them).  Returns the member count (uniform).
// Ends with a barrier.
__device__ __forceinline__ uint32_t compact_members(FastShared &sh) {
  const int tid = threadIdx.x;
  constexpr int kPer = kHashCap / kFT;
  const uint32_t *hkeys = sh.u32(0), *hcnt = sh.u32(kHashCap * 4);
  uint32_t *midx = sh.m_idx(), *mkey = sh.m_key();
  // thread t owns slots t, t + kFT, ...: conflict-free reads, all in flight at once
  uint32_t keys[kPer];
  uint32_t n = 0, nmem;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    keys[i] = hkeys[tid + i * kFT];
    n += keys[i] ? 1u : 0u;
  }
  const uint32_t off = block_exclusive_scan<kFW>(n, sh.uscr, &nmem);
  if (nmem <= (uint32_t)kFastMembers) {
    uint32_t o = off;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      if (keys[i]) {
        midx[o] = keys[i] - 1u;
        mkey[o] = hcnt[tid + i * kFT];
        ++o;
      }
    }
  }
  __syncthreads();
  return nmem;
}

// This thread's history ids (strided by the block; positions past the end
// re-read the first id and are ignored by insert_history).
__device__ __forceinline__ void load_history_ids(uint32_t (&hid)[kHistPer], const lmrs_sample_args &a,
                                                 const RowCfg &c) {
#pragma unroll
  for (int q = 0; q < kHistPer; ++q) {
    const int64_t j = (int64_t)threadIdx.x + (int64_t)q * kFT;
    hid[q] = a.hist_ids[c.h_begin + (j < c.h_len ? j : 0)];
  }
}

// The same loads, issued (not waited for) as explicit instructions.
__device__ __forceinline__ void issue_history_ids(uint32_t (&hid)[kHistPer], const lmrs_sample_args &a,
                                                  const RowCfg &c) {
#pragma unroll
  for (int q = 0; q < kHistPer; ++q) {
    const int64_t j = (int64_t)threadIdx.x + (int64_t)q * kFT;
    hid[q] = issue_load_b32(a.hist_ids + c.h_begin + (j < c.h_len ? j : 0));
  }
}

// Raw logits of the members (one load each, a fixed number per thread).
__device__ __forceinline__ void load_member_raw(uint32_t (&mraw)[kMemPer], FastShared &sh, uint32_t nmem,
                                                const uint16_t *rowp) {
  const uint32_t *midx = sh.m_idx();
#pragma unroll
  for (int q = 0; q < kMemPer; ++q) {
    const uint32_t m = (uint32_t)threadIdx.x + (uint32_t)q * kFT;
    mraw[q] = rowp[m < nmem ? midx[m] : 0u];
  }
}

// The same loads, issued (not waited for) as explicit instructions.
__device__ __forceinline__ void issue_member_raw(uint32_t (&mraw)[kMemPer], FastShared &sh, uint32_t nmem,
                                                 const uint16_t *rowp) {
  const uint32_t *midx = sh.m_idx();
#pragma unroll
  for (int q = 0; q < kMemPer; ++q) {
    const uint32_t m = (uint32_t)threadIdx.x + (uint32_t)q * kFT;
    mraw[q] = issue_load_u16(rowp + (m < nmem ? midx[m] : 0u));
  }
}

// Member keys: m_key[m] = raw key | z key << 16.  Returns this thread's
// largest member z key; *bad is set when a z is a NaN.
__device__ __forceinline__ uint32_t member_keys(FastShared &sh, const uint32_t (&mraw)[kMemPer], uint32_t nmem,
                                                const RowCfg &c, uint32_t *bad) {
  uint32_t *mkey = sh.m_key();
  uint32_t zmax = 0u;
#pragma unroll
  for (int q = 0; q < kMemPer; ++q) {
    const uint32_t m = (uint32_t)threadIdx.x + (uint32_t)q * kFT;
    if (m < nmem) {
      const uint32_t zk = bits_key16(penalise_member(mraw[q], mkey[m], c));
      mkey[m] = bits_key16(mraw[q]) | (zk << 16);
      zmax = max(zmax, zk);
      *bad |= is_nan_key16(zk) ? 1u : 0u;
    }
  }
  return zmax;
}

// Rebuilds the member list and bitmap (after the full path reused their
// space), with the raw logits fetched again.  Ends with a barrier.
__device__ __forceinline__ void rebuild_members(FastShared &sh, const lmrs_sample_args &a, const RowCfg &c,
                                                int64_t V, const uint16_t *rowp) {
  uint32_t hid[kHistPer];
  load_history_ids(hid, a, c);
  clear_history(sh);
  insert_history(sh, hid, c.h_len, V);
  const uint32_t nmem = compact_members(sh);
  uint32_t mraw[kMemPer], bad = 0u;
  load_member_raw(mraw, sh, nmem, rowp);
  member_keys(sh, mraw, nmem, c, &bad);
  __syncthreads();
}

// ---- selection over LDS data ------------------------------------------------------

// Chunk maxima of this thread's NCH chunk slots, two 16-bit keys per word
// (slot s in the low half of cm[s / 2] when s is even).  They stay in
// registers: every pass that filters on them reads them without latency.
template <int NCH>
struct ChunkMax {
  uint32_t w[(NCH + 1) / 2];
  __device__ __forceinline__ uint32_t get(int s) const { return (w[s >> 1] >> ((s & 1) * 16)) & 0xFFFFu; }
};

// The K-th largest value among the chunk maxima of the chunks without
// history tokens (bit s of `mixed` set: slot s holds one) and the member z
// keys -- each value stands for a distinct element whose z is at least the
// value -- by a cascade of windows below `hi`, each twice as wide as the
// last.  Returns false (uniformly) when fewer than K values exist.
template <int NCH>
__device__ __forceinline__ bool kth_value(FastShared &sh, const ChunkMax<NCH> &cm, bool roww, uint64_t mixed,
                                          uint32_t nmem, uint32_t K, uint32_t hi, uint32_t *out) {
  const int tid = threadIdx.x;
  const uint32_t *mkey = sh.m_key();
  uint32_t *wh = sh.whist();
  uint32_t above = 0u, w = 64u;
  for (;;) {
    const uint32_t lo = hi >= w - 1u ? hi - (w - 1u) : 0u;
    const uint32_t nbins = hi - lo + 1u;
    for (uint32_t i = tid; i < nbins; i += kFT) wh[i] = 0u;
    __syncthreads();
    if (roww) {
#pragma unroll
      for (int s = 0; s < NCH; ++s) {
        const uint32_t v = cm.get(s);
        if (!((mixed >> s) & 1u) && v >= lo && v <= hi) atomicAdd(&wh[v - lo], 1u);
      }
    }
    for (uint32_t m = tid; m < nmem; m += kFT) {
      const uint32_t z = mkey[m] >> 16;
      if (z >= lo && z <= hi) atomicAdd(&wh[z - lo], 1u);
    }
    __syncthreads();
    const uint32_t mine = (uint32_t)tid < nbins ? wh[nbins - 1u - (uint32_t)tid] : 0u;  // bin hi - tid
    uint32_t wtot;
    const uint32_t ex = block_exclusive_scan<kFW>(mine, sh.uscr, &wtot);
    if (above + wtot >= K) {
      if (mine > 0u && above + ex < K && K <= above + ex + mine) sh.bsel[0] = hi - (uint32_t)tid;
      __syncthreads();
      *out = uniform(sh.bsel[0]);
      return true;
    }
    if (lo == 0u) return false;
    above += wtot;
    hi = lo - 1u;
    w = min(w * 2u, (uint32_t)kMaxWindow);
  }
}

// Exact finish over the sorted candidates held one per lane of a wave (lane
// i holds the i-th entry (~ykey << 32 | index), k <= 64 entries):
// f64 weights exp(f64(l - max)), DPP prefix sums, the nucleus cut
// (top_p.rs:45-58) and softmax_choice (strategies/mod.rs:27-55).
template <class TR>
__device__ __forceinline__ void finish_wave(uint64_t g, const RowCfg &c, const lmrs_sample_args &a, int r,
                                            uint32_t k, bool greedy) {
  const uint32_t lane = threadIdx.x & 63u;
  const bool in = lane < k;
  const float y = TR::value(~(uint32_t)(g >> 32));
  const float M = TR::value(~(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(g >> 32), 0));
  const double w = in ? exp((double)(y - M)) : 0.0;
  const double incl = wave_inclusive<OpSum>(w, 0.0);
  const double total = lane63(incl);
  if (!(__builtin_isfinite(total) && total > 0.0)) {
    if (lane == 0) write_row(a, r, 0u, 0.0f, 0.0f, LMRS_ROW_DISTRIBUTION);
    return;
  }
  uint32_t keep = k;
  int32_t flags = 0;
  if (c.top_p < 1.0 && !greedy) {  // Greedy applies no nucleus cut (greedy.rs:22-29)
    const double acc = incl / total;
    const uint64_t hit = __ballot(in && acc >= c.top_p);
    if (hit) keep = (uint32_t)__builtin_ctzll(hit) + 1u;
    // nucleus margin at the cut, from the lane of entry keep - 1
    const double prev = (incl - w) / total;
    double m = c.top_p - prev;
    if (acc >= c.top_p && acc - c.top_p < m) m = acc - c.top_p;
    if (!(acc >= c.top_p)) m = c.top_p - acc;
    const uint64_t near = __ballot(lane + 1u == keep && m < 1e-6);
    if (near) flags |= LMRS_ROW_NEAR_BOUNDARY;
  }
  const uint64_t ib = (uint64_t)__double_as_longlong(incl);
  const uint32_t klo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)ib, (int)(keep - 1u));
  const uint32_t khi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(ib >> 32), (int)(keep - 1u));
  const double sum_keep = __longlong_as_double((long long)(((uint64_t)khi << 32) | klo));
  const double target = c.u * sum_keep;
  const uint64_t pickm = __ballot(lane < keep && target <= incl);
  const uint32_t pick = pickm ? (uint32_t)__builtin_ctzll(pickm) : keep - 1u;  // fallback: last (mod.rs:52-54)
  if (lane == pick) {
    const double lo = (incl - w) / sum_keep, hi = incl / sum_keep;
    double m = 1.0;
    if (pick > 0u && fabs(c.u - lo) < m) m = fabs(c.u - lo);
    if (pick + 1u < keep && fabs(hi - c.u) < m) m = fabs(hi - c.u);
    write_row(a, r, (uint32_t)(g & 0xFFFFFFFFu), (float)log(w / sum_keep), y,
              flags | (m < 1e-6 ? LMRS_ROW_NEAR_BOUNDARY : 0));
  }
}

// ---- the ordered search of the full path ------------------------------------------

// Net count change of a member for the range [lo, hi]: it leaves its raw key
// and enters at its z key.
__device__ __forceinline__ int member_delta(uint32_t mk, uint32_t lo, uint32_t hi) {
  const uint32_t rk = mk & 0xFFFFu, zk = mk >> 16;
  return (zk >= lo && zk <= hi ? 1 : 0) - (rk >= lo && rk <= hi ? 1 : 0);
}

// Elements of a chunk (raw bf16 words) with a raw key in [lo, hi] (members
// are corrected by the caller).
__device__ __forceinline__ uint32_t chunk_matches(const uint4 &d, uint32_t lo, uint32_t hi) {
  const uint32_t w[4] = {key_pair(d.x), key_pair(d.y), key_pair(d.z), key_pair(d.w)};
  uint32_t n = 0u;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t key = (w[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
    n += (key >= lo && key <= hi) ? 1u : 0u;
  }
  return n;
}

// The j-th (1-based) lowest index among elements whose z key lies in [lo, hi]
// (members by their z key), on a second read of the row.  Index order is
// (slot, thread, element): per-slot match counts are reduced into LDS, the
// slot holding the j-th match is found, and one block scan over that slot's
// per-thread counts locates the chunk and then the element.
template <int NCH>
__device__ __forceinline__ uint32_t find_jth_stream(FastShared &sh, const uint4 *src, int nchunks, uint32_t nmem,
                                                    uint32_t lo, uint32_t hi, uint32_t j) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool roww = wave >= kHW;
  const int rt = tid - 64 * kHW, rw = wave - kHW;  // row thread and row wave
  uint32_t *slot_cnt = sh.u32(kOffSlotCnt), *tcnt = sh.u32(kOffTcnt);
  const uint32_t *midx = sh.m_idx(), *mkey = sh.m_key();
  for (int i = tid; i < NCH * kRW; i += kFT) slot_cnt[i] = 0u;
  __syncthreads();
  if (roww) {
    constexpr int G = 8;  // slots in flight at a time
    const int ft = fresh_tid() - 64 * kHW;
#pragma unroll
    for (int s0 = 0; s0 < NCH; s0 += G) {
      uint4 d[G];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int ch = (s0 + g) * kRT + ft;
        if (s0 + g < NCH) d[g] = *(ch < nchunks ? src + ch : &kNegInfChunk);
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int s = s0 + g;
        if (s < NCH) {
          const uint32_t n = (s * kRT + ft < nchunks) ? chunk_matches(d[g], lo, hi) : 0u;
          const uint32_t t = wave_sum(n);
          if (lane == 0 && t) atomicAdd(&slot_cnt[s * kRW + rw], t);
        }
      }
    }
  }
  for (uint32_t m = tid; m < nmem; m += kFT) {
    const int dl = member_delta(mkey[m], lo, hi);
    const uint32_t ch = midx[m] >> 3;
    if (dl) atomicAdd(&slot_cnt[(ch / kRT) * kRW + ((ch % kRT) >> 6)], (uint32_t)dl);
  }
  __syncthreads();
  if (tid < NCH) {  // per-slot totals
    uint32_t tot = 0;
    for (int w = 0; w < kRW; ++w) tot += slot_cnt[tid * kRW + w];
    tcnt[tid] = tot;
  }
  __syncthreads();
  if (tid == 0) {
    uint32_t acc = 0, sstar = NCH - 1, before = 0;
    for (int s = 0; s < NCH; ++s) {
      const uint32_t tot = tcnt[s];
      if (acc + tot >= j) {
        sstar = (uint32_t)s;
        before = acc;
        break;
      }
      acc += tot;
    }
    sh.bsel[0] = sstar;
    sh.bsel[1] = before;
  }
  __syncthreads();
  const int sstar = (int)uniform(sh.bsel[0]);
  const uint32_t jr = j - uniform(sh.bsel[1]);
  if (roww) tcnt[rt] = 0u;
  if (tid < 8) sh.chunk_z[tid] = 0xFFFFFFFFu;
  __syncthreads();
  for (uint32_t m = tid; m < nmem; m += kFT) {  // members of slot sstar, per owner row thread
    const int dl = member_delta(mkey[m], lo, hi);
    const uint32_t ch = midx[m] >> 3;
    if (dl && (int)(ch / kRT) == sstar) atomicAdd(&tcnt[ch % kRT], (uint32_t)dl);
  }
  __syncthreads();
  const int chs = sstar * kRT + rt;
  uint32_t mine = 0u;
  if (roww) {
    mine = tcnt[rt];
    if (chs < nchunks) mine += chunk_matches(src[chs], lo, hi);
  }
  uint32_t tot;
  const uint32_t excl = block_exclusive_scan<kFW>(mine, sh.uscr, &tot);  // wave 0 adds zeros first
  if (roww && excl < jr && jr <= excl + mine) {
    sh.bsel[2] = (uint32_t)chs;  // the chunk
    sh.bsel[3] = jr - excl;      // rank inside it
  }
  __syncthreads();
  const uint32_t cstar = uniform(sh.bsel[2]), need0 = uniform(sh.bsel[3]);
  for (uint32_t m = tid; m < nmem; m += kFT)
    if ((midx[m] >> 3) == cstar) sh.chunk_z[midx[m] & 7u] = mkey[m] >> 16;
  __syncthreads();
  if (tid == 0) {
    const uint4 dd = src[min(cstar, (uint32_t)nchunks - 1u)];  // (thread 0 reads the chosen chunk)
    const uint4 w = make_uint4(key_pair(dd.x), key_pair(dd.y), key_pair(dd.z), key_pair(dd.w));
    uint32_t need = need0, pick = cstar * 8u;
    for (uint32_t e = 0; e < 8u; ++e) {
      const uint32_t zm = sh.chunk_z[e];
      const uint32_t key = zm != 0xFFFFFFFFu ? zm : chunk_key(w, e);
      if (key >= lo && key <= hi) {
        if (need == 1u) {
          pick = cstar * 8u + e;
          break;
        }
        need -= 1u;
      }
    }
    sh.bsel[4] = pick;
  }
  __syncthreads();
  const uint32_t idx = uniform(sh.bsel[4]);
  __syncthreads();
  return idx;
}

// ---- one row ----------------------------------------------------------------------

// Returns false (uniformly) when the row must go to the generic engine,
// before any output of the row is written.
template <int NCH>
__device__ __forceinline__ bool fast_row(FastShared &sh, const lmrs_sample_args &a, int r) {
  using TR = DTypeTraits<LMRS_DTYPE_BF16>;
  const int tid = threadIdx.x, wave = tid >> 6;
  const bool roww = wave >= kHW;  // row thread
  const int rt = tid - 64 * kHW;  // row thread index
  const int64_t V = a.vocab;
  const int nchunks = (int)(V >> 3);
  const uint32_t npad = (uint32_t)(NCH * kRT - nchunks) * 8u;
  const uint16_t *rowp = (const uint16_t *)((const char *)a.logits + (size_t)r * (size_t)a.row_stride * 2);
  const uint4 *src = (const uint4 *)rowp;
  u32x4 kv[NCH];
  uint32_t k[NCH][4];

  // Parameters through scalar loads (no store precedes them).  Then, in this
  // order: the history ids (requests queue in issue order across the whole
  // chip: ids requested after 64 MB of logits would arrive after them), the
  // first quarter of the row, the member build (hash, bitmap, member list)
  // while that quarter streams in, the members' raw logits, the rest of the
  // row.  A wave issuing loads faster than memory drains them stalls at the
  // issue, so work placed after the last load would wait for most of the row.
  // No path leaves before the load pass consumes the row.
  const RowCfg c = uniform_cfg(load_row_cfg(a, r, LMRS_DTYPE_BF16));
  const bool hist = c.status == LMRS_ROW_OK && c.hist_on;
  constexpr int kEarly = NCH / 4;
  uint32_t hid[kHistPer];
  if (hist) issue_history_ids(hid, a, c);
  if (roww) {
#pragma unroll
    for (int s = 0; s < kEarly; ++s) {
      const int ch = s * kRT + rt;
      kv[s] = issue_load_b128(ch < nchunks ? src + ch : &kNegInfChunk);  // lanes past the end load -inf
    }
  }
  uint32_t nmem = 0u;
  uint32_t mraw[kMemPer];
  if (hist) {
    clear_history(sh);
#pragma unroll
    for (int q = 0; q < kHistPer; ++q) wait_loads<kEarly>(hid[q]);  // the first quarter stays in flight
    insert_history(sh, hid, c.h_len, V);
    nmem = compact_members(sh);
    issue_member_raw(mraw, sh, nmem <= (uint32_t)kFastMembers ? nmem : 0u, rowp);
  }
  if (roww) {
#pragma unroll
    for (int s = kEarly; s < NCH; ++s) {
      const int ch = s * kRT + rt;
      kv[s] = issue_load_b128(ch < nchunks ? src + ch : &kNegInfChunk);
    }
  }

  // The load pass: raw keys, chunk maxima (all elements), the NaN check, and
  // which elements are history tokens (8 bits per chunk, four chunks a word).
  const uint32_t *bitmap = sh.bitmap();
  ChunkMax<NCH> cm;
  uint32_t hbits[(NCH + 3) / 4];
  uint64_t mixed = 0u;
  uint32_t mx = 0u, mn = 0xFFFFFFFFu, bad = 0u;
  if (roww) {
    static_for<0, NCH>([&](auto S) {
      constexpr int s = decltype(S)::value;
      const int ch = s * kRT + rt;
      wait_loads<NCH - 1 - s>(kv[s]);  // exact for the later loads, conservative for the first quarter
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t kp = key_pair(kv[s][q]);
        k[s][q] = kp;
        mn = pk_min_u16(mn, kp);
      }
      uint32_t cmx = chunk_max(k[s]);
      bad |= cmx >= 0xFF81u ? 1u : 0u;
      const bool valid = (s + 1) * kRT <= nchunks || ch < nchunks;
      if (!valid) cmx = 0u;  // padding: no candidates
      cm.w[s >> 1] = (s & 1) ? (cm.w[s >> 1] | (cmx << 16)) : cmx;
      mx = max(mx, cmx);
      uint32_t m8 = 0u;
      if (hist && valid) m8 = (bitmap[ch >> 2] >> ((ch & 3) * 8)) & 0xFFu;
      hbits[s >> 2] = (s & 3) ? (hbits[s >> 2] | (m8 << ((s & 3) * 8))) : m8;
      mixed |= (uint64_t)(m8 != 0u) << s;
    });
    bad |= min(mn & 0xFFFFu, mn >> 16) <= 0x007Eu ? 1u : 0u;
  }
  if (hist && nmem <= (uint32_t)kFastMembers) {
#pragma unroll
    for (int q = 0; q < kMemPer; ++q) wait_loads<0>(mraw[q]);
    mx = max(mx, member_keys(sh, mraw, nmem, c, &bad));
  }
  if (c.status != LMRS_ROW_OK) {
    if (tid == 0) write_row(a, r, 0u, 0.0f, 0.0f, c.status);
    return true;
  }
  if (nmem > (uint32_t)kFastMembers) return false;
  block_max2(mx, bad, sh);
  // Rows with a NaN go to the generic engine: the processors canonicalise
  // NaNs, which the key map does not model.
  if (bad) return false;
  const uint32_t ztop = mx;  // no z key of the row is larger
  const bool k_on = c.top_k > 0 && c.top_k < V;
  const uint32_t *midx = sh.m_idx(), *mkey = sh.m_key();
  const uint4 *src2 = fresh(src);  // the re-reads of the full path

  if (k_on && c.top_k <= kGatherCap) {  // ---- greedy and small k ----------------------
    // Greedy (greedy.rs:22-29) is the case k = 1: the first of the sorted candidates.
    const uint32_t K = (uint32_t)c.top_k;
    uint32_t L;
    if (!kth_value(sh, cm, roww, mixed, nmem, K, ztop, &L)) return false;
    const uint32_t za = group_low(L, c);
    // gather every element with z >= za: (~(y key << 16) << 32 | index).
    // Count first (8-bit masks per candidate chunk, packed four to a word),
    // then one scan gives every thread its write offset: no atomics.
    SelState &ss = sh.ss();
    uint32_t masks[(NCH + 3) / 4];
    uint32_t nmine = 0u;
    static_for<0, NCH>([&](auto S) {
      constexpr int s = decltype(S)::value;
      uint32_t m8 = 0u;
      if (roww && cm.get(s) >= za) {
#pragma unroll
        for (int e = 0; e < 8; ++e) m8 |= (((k[s][e >> 1] >> ((e & 1) * 16)) & 0xFFFFu) >= za ? 1u : 0u) << e;
        m8 &= ~(hbits[s >> 2] >> ((s & 3) * 8)) & 0xFFu;  // members enter by their z key
      }
      masks[s >> 2] = (s & 3) ? (masks[s >> 2] | (m8 << ((s & 3) * 8))) : m8;
      nmine += (uint32_t)__builtin_popcount(m8);
    });
    for (uint32_t m = tid; m < nmem; m += kFT) nmine += (mkey[m] >> 16) >= za ? 1u : 0u;
    uint32_t ncand;
    uint32_t pos = block_exclusive_scan<kFW>(nmine, sh.uscr, &ncand);
    if (ncand <= (uint32_t)kGatherCap) {
      static_for<0, NCH>([&](auto S) {
        constexpr int s = decltype(S)::value;
        uint32_t m8 = (masks[s >> 2] >> ((s & 3) * 8)) & 0xFFu;
        if (m8) {
          const uint32_t ch = (uint32_t)(s * kRT + rt);
          const uint4 w = make_uint4(k[s][0], k[s][1], k[s][2], k[s][3]);
          do {
            const uint32_t e = (uint32_t)__builtin_ctz(m8);
            m8 &= m8 - 1u;
            ss.gather[pos++] = ((uint64_t)(~(temp_key16(chunk_key(w, e), c) << 16)) << 32) | (ch * 8u + e);
          } while (m8);
        }
      });
      for (uint32_t m = tid; m < nmem; m += kFT) {
        const uint32_t zk = mkey[m] >> 16;
        if (zk >= za) ss.gather[pos++] = ((uint64_t)(~(temp_key16(zk, c) << 16)) << 32) | midx[m];
      }
    }
    __syncthreads();
    if (ncand > (uint32_t)kGatherCap) return false;
    if (ncand <= 64u) {
      // rank sort inside wave 0: entry i moves to lane (number of smaller entries)
      if (tid < 64) {
        const uint64_t g = (uint32_t)tid < ncand ? ss.gather[tid] : ~0ull;
        uint32_t rank = 0u;
#pragma unroll 8
        for (uint32_t j = 0; j < ncand; ++j) rank += ss.gather[j] < g ? 1u : 0u;
        if ((uint32_t)tid >= ncand) rank = (uint32_t)tid;
        const uint32_t lo32 = (uint32_t)__builtin_amdgcn_ds_permute((int)(rank * 4u), (int)(uint32_t)g);
        const uint32_t hi32 = (uint32_t)__builtin_amdgcn_ds_permute((int)(rank * 4u), (int)(uint32_t)(g >> 32));
        finish_wave<TR>(((uint64_t)hi32 << 32) | lo32, c, a, r, K, K == 1u);
      }
      return true;
    }
    sort_gather<kFT>(ss, ncand);
    finish_sorted<TR, kFT>(ss, c, a, r, K);
    return true;
  }

  // ---- full: 65536-bin count histogram ------------------------------------------
  __syncthreads();  // the hash, bitmap and window views are dead
  uint32_t *h64 = sh.u32(0);
  {
    uint4 *p = (uint4 *)h64;
    for (int i = tid; i < 8192; i += kFT) p[i] = make_uint4(0u, 0u, 0u, 0u);
  }
  __syncthreads();
  auto count_word = [&](uint32_t w) {
    const uint32_t ka = w & 0xFFFFu, kb = w >> 16;
    atomicAdd(&h64[ka & 0x7FFFu], (ka & 0x8000u) ? 0x10000u : 1u);
    atomicAdd(&h64[kb & 0x7FFFu], (kb & 0x8000u) ? 0x10000u : 1u);
  };
  if (roww) {
#pragma unroll
    for (int s = 0; s < NCH; ++s) {
#pragma unroll
      for (int q = 0; q < 4; ++q) count_word(k[s][q]);
    }
  }
  __syncthreads();
  // members move from their raw key to their z key; padding leaves -inf
  for (uint32_t m = tid; m < nmem; m += kFT) {
    const uint32_t zk = mkey[m] >> 16;
    atomicAdd(&h64[zk & 0x7FFFu], (zk & 0x8000u) ? 0x10000u : 1u);
  }
  __syncthreads();
  for (uint32_t m = tid; m < nmem; m += kFT) {
    const uint32_t rk = mkey[m] & 0xFFFFu;
    atomicSub(&h64[rk & 0x7FFFu], (rk & 0x8000u) ? 0x10000u : 1u);
  }
  if (tid == 0) atomicSub(&h64[kNegInfKey16], npad);
  __syncthreads();
  // Compaction.  Thread t owns the KPT keys 65535-KPT*t .. 65536-KPT*(t+1)
  // (descending; position j holds key 65535-KPT*t-j): the high halves of
  // words 32767-KPT*t-j for the first half of the threads, else the low
  // halves.  Reads are rotated by the thread id so that the lanes of a wave
  // hit different banks.
  constexpr int KPT = 65536 / kFT, NM = KPT / 64;
  const int wbase = 32767 - KPT * (tid & (kFT / 2 - 1));
  const int hsh = tid < kFT / 2 ? 16 : 0;
  uint64_t nz[NM];
#pragma unroll
  for (int i = 0; i < NM; ++i) nz[i] = 0;
  uint32_t csum = 0;
  for (int jj = 0; jj < KPT; ++jj) {
    const int j = (jj + tid) & (KPT - 1);
    const uint32_t cn = (h64[wbase - j] >> hsh) & 0xFFFFu;
    csum += cn;
#pragma unroll
    for (int i = 0; i < NM; ++i)
      if ((j >> 6) == i) nz[i] |= (uint64_t)(cn != 0u) << (j & 63);
  }
  uint32_t nbins, nzc = 0;
#pragma unroll
  for (int i = 0; i < NM; ++i) nzc += (uint32_t)__builtin_popcountll(nz[i]);
  const uint32_t eoff = block_exclusive_scan<kFW>(nzc, sh.uscr, &nbins);
  const uint32_t total = block_sum<kFW>(csum, sh.uscr);
  // a key with more than 65535 elements, or too many distinct keys
  if (total != (uint32_t)V || nbins > (uint32_t)kMaxEntries) return false;
  // entries (key << 16 | count) in descending key order, outside the counters
  uint32_t *ent = sh.u32(kOffEntries);
  for (int jj = 0; jj < KPT; ++jj) {
    const int j = (jj + tid) & (KPT - 1);
    const uint32_t cn = (h64[wbase - j] >> hsh) & 0xFFFFu;
    if (cn) {
      uint32_t below = 0;
#pragma unroll
      for (int i = 0; i < NM; ++i) {
        if ((j >> 6) > i) below += (uint32_t)__builtin_popcountll(nz[i]);
        if ((j >> 6) == i) below += (uint32_t)__builtin_popcountll(nz[i] & ((1ull << (j & 63)) - 1ull));
      }
      ent[eoff + below] = ((uint32_t)(65535 - KPT * tid - j) << 16) | cn;
    }
  }
  __syncthreads();  // the counters are dead: their space holds the prefixes
  double *mincl = (double *)sh.u32(0);        // inclusive mass prefix
  uint32_t *cincl = sh.u32(kMaxEntries * 8);  // inclusive count prefix
  const int nb = (int)nbins;
  const int E = (nb + kFT - 1) / kFT;  // entries per thread, contiguous
  const float M = key16_value(temp_key16(ent[0] >> 16, c));
  // per-token weight exp(f64(y - max)) of entry e (strategies/mod.rs:35)
  auto weight_of = [&](int e) { return exp((double)(key16_value(temp_key16(ent[e] >> 16, c)) - M)); };
  uint32_t lc = 0;
  double lm = 0.0;
  for (int i = 0; i < E; ++i) {
    const int e = tid * E + i;
    if (e < nb) {
      const uint32_t cn = ent[e] & 0xFFFFu;
      lc += cn;
      lm += (double)cn * weight_of(e);
    }
  }
  uint32_t ctot;
  double mtot;
  const uint32_t cex = block_exclusive_scan<kFW>(lc, sh.uscr, &ctot);
  const double mex = block_exclusive_scan<kFW>(lm, sh.dscr, &mtot);
  lc = cex;
  lm = mex;
  for (int i = 0; i < E; ++i) {
    const int e = tid * E + i;
    if (e < nb) {
      const uint32_t cn = ent[e] & 0xFFFFu;
      lc += cn;
      lm += (double)cn * weight_of(e);
      cincl[e] = lc;
      mincl[e] = lm;
    }
  }
  __syncthreads();
  // Tie groups: runs of entries (descending z) with equal y.
  auto ykey_of = [&](int e) { return temp_key16(ent[e] >> 16, c); };
  auto group_head = [&](int e) {
    const uint32_t y = ykey_of(e);
    while (e > 0 && ykey_of(e - 1) == y) --e;
    return e;
  };
  auto group_tail = [&](int e) {
    const uint32_t y = ykey_of(e);
    while (e + 1 < nb && ykey_of(e + 1) == y) ++e;
    return e;
  };
  auto cnt_excl = [&](int e) { return cincl[e] - (ent[e] & 0xFFFFu); };
  auto mass_excl = [&](int e) { return mincl[e] - (double)(ent[e] & 0xFFFFu) * weight_of(e); };
  // First entry (<= last) whose inclusive prefix reaches the target; -1 if none.
  auto first_mass = [&](double target, int last) {
    int f = 0x7FFFFFFF;
    for (int i = E - 1; i >= 0; --i) {
      const int e = tid * E + i;
      if (e < nb && e <= last && mincl[e] >= target) f = e;
    }
    f = block_min<kFW>(f, sh.iscr);
    return f == 0x7FFFFFFF ? -1 : f;
  };
  auto first_count = [&](uint32_t target) {
    int f = 0x7FFFFFFF;
    for (int i = E - 1; i >= 0; --i) {
      const int e = tid * E + i;
      if (e < nb && cincl[e] >= target) f = e;
    }
    return block_min<kFW>(f, sh.iscr);
  };

  // candidates: the top-k cut at tie-group granularity
  int last_e = nb - 1;  // last entry holding kept tokens
  int last_h = group_head(last_e);
  uint32_t last_keep = ctot - cnt_excl(last_h);  // kept tokens of the last group
  double cand_mass = mtot;
  if (k_on) {
    const int f = first_count((uint32_t)c.top_k);
    last_h = group_head(f);
    last_e = group_tail(f);
    last_keep = (uint32_t)c.top_k - cnt_excl(last_h);
    cand_mass = mass_excl(last_h) + (double)last_keep * weight_of(last_h);
  }
  int32_t flags = 0;
  double kept_mass = cand_mass;
  if (c.top_p < 1.0) {
    // nucleus cut (top_p.rs:45-58) over the candidates
    const double tp = c.top_p * cand_mass;
    const int f = first_mass(tp, last_e);
    if (f >= 0) {
      const int h = group_head(f), t = group_tail(f);
      const double wg = weight_of(h), mx2 = mass_excl(h);
      const uint32_t gmax = (h == last_h) ? last_keep : cincl[t] - cnt_excl(h);
      double jj = ceil((tp - mx2) / wg);
      if (!(jj >= 1.0)) jj = 1.0;
      if (jj > (double)gmax) jj = (double)gmax;
      const uint32_t jp = (uint32_t)jj;
      kept_mass = mx2 + (double)jp * wg;
      const double acc = kept_mass / cand_mass, prev = (kept_mass - wg) / cand_mass;
      double m = c.top_p - prev;
      if (acc - c.top_p < m) m = acc - c.top_p;
      if (m < 1e-6) flags |= LMRS_ROW_NEAR_BOUNDARY;
      last_h = h;
      last_e = t;
      last_keep = jp;
    } else if (c.top_p - 1.0 > -1e-6) {
      flags |= LMRS_ROW_NEAR_BOUNDARY;
    }
  }
  // the draw (softmax_choice, strategies/mod.rs:44-54)
  const double target = c.u * kept_mass;
  int f = first_mass(target, last_e);
  const bool ovf = f < 0;
  if (ovf) f = last_e;
  const int h = group_head(f), tl = group_tail(f);
  const double mx2 = mass_excl(h), wg = weight_of(h);
  const uint32_t gmax = (h == last_h) ? last_keep : cincl[tl] - cnt_excl(h);
  double jj = ovf ? (double)gmax : ceil((target - mx2) / wg);
  if (!(jj >= 1.0)) jj = 1.0;
  if (jj > (double)gmax) jj = (double)gmax;
  const uint32_t jt = (uint32_t)jj;
  const uint32_t zhi = uniform(ent[h] >> 16), zlo = uniform(ent[tl] >> 16);
  const float yv = key16_value(ykey_of(h));
  const bool first_tok = (h == 0 && jt == 1u), last_tok = (h == last_h && jt == gmax);
  __syncthreads();  // entries and prefixes are dead
  if (nmem) rebuild_members(sh, a, c, V, rowp);
  const uint32_t token = find_jth_stream<NCH>(sh, src2, nchunks, nmem, zlo, zhi, jt);
  if (tid == 0) {
    const double lo_c = (mx2 + (double)(jt - 1u) * wg) / kept_mass, hi_c = lo_c + wg / kept_mass;
    double m = 1.0;
    if (!first_tok && fabs(c.u - lo_c) < m) m = fabs(c.u - lo_c);
    if (!last_tok && fabs(hi_c - c.u) < m) m = fabs(hi_c - c.u);
    if (ovf) m = 0.0;
    write_row(a, r, token, (float)log(wg / kept_mass), yv, flags | (m < 1e-6 ? LMRS_ROW_NEAR_BOUNDARY : 0));
  }
  return true;
}

template <int NCH>
__global__ void __launch_bounds__(kFT) bf16_fast_kernel(lmrs_sample_args a) {
  __shared__ FastOrGeneric sh;
  const int r = blockIdx.x;
  if (fast_row<NCH>(sh.f, a, r)) return;
  __syncthreads();
  generic_row<LMRS_DTYPE_BF16, kFT>(sh.g, a, r, 1);
}

}  // namespace lmrs
