// fast_bf16.hpp -- the bf16 sampling kernel for rows of up to kFastMaxVocab.
//
// One workgroup of 512 threads (one per CU at this LDS size; 8 waves, so each
// thread may hold 256 VGPRs) owns one row.  Each thread loads its NCH 16-byte
// chunks (chunk c = s * 512 + thread, slot s = 0 .. NCH-1) with explicitly
// issued loads and keeps them in registers as 16-bit total-order keys of the
// RAW logits, two per word: the row is read from memory once.
//
// History.  The history ids are requested right after the row's first two
// slots and the row parameters.  Inside the load pass,
// after slot kHistAt, they are marked in an LDS bitmap over the vocab; the
// number of marked tokens before each 32-token bitmap word gives every
// distinct history token ("member", at most kFastMembers) a dense index in
// token order, under which its multiplicity is counted; each member's raw
// logit is then requested with one 16-bit load, and kEarly + 1 slots later
// its penalised key z (Repetition then Presence/Frequency, bf16-rounded per
// op, as the reference's chain of kernels) is computed.  The bitmap also
// tells which chunks hold members.
// Temperature is not applied per element either: y = bf16(fma(z, 1/T, 0)) is
// monotone in z, so selection runs on z keys and maps only the keys that
// matter to y; runs of z keys that round to one y form one tie group, whose
// tokens are ordered by index as the reference's sort orders them.
//
// Paths after the load pass:
//   small k  (top_k <= kSmallK, greedy included): every thread holds one
//            "thread value": its largest chunk maximum when that chunk holds
//            no member (else none), raised to its members' z keys -- each a
//            distinct element's key.  The K-th largest thread value L (LDS
//            histograms) bounds the K-th largest z from below.  Every
//            element at or above the start of L's tie group is a candidate:
//            those of the thread's largest chunk, whose keys the load pass
//            kept, of its other chunks whose maximum reaches the bound (rare;
//            from registers) and the members.  Up to 64 candidates are
//            ranked across the waves and finished by one wave in f64; up to
//            512 ranked by one thread each; more are sorted in LDS.
//   window   (top_k = 0 or > kSmallK): a 512-bin LDS histogram of the keys
//            within 512 of the maximum, every other element's weight summed
//            in f32 (chunks whose weights are all below e^-37 skipped); the
//            window's keys carry exact f64 weights and counts for the top-k,
//            min-p and nucleus cuts and the draw; the chosen token is the
//            j-th lowest index of its tie group, found in registers.  A cut
//            or target below a window whose tail still carries mass declines
//            to the next path.
//   mid k    (top_k <= kGatherCap): the same bound from the K-th largest
//            chunk maximum (a cascade of LDS windows), the candidates
//            gathered from registers and sorted in LDS.
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
constexpr int kMaxEntries = 6144;   // distinct keys the full path keeps in LDS
constexpr int kFastMembers = 2048;  // distinct history tokens the fast path keeps
constexpr int kMaxSlots = 40;       // chunk slots per thread
constexpr int kFastMaxVocab = kMaxSlots * 8 * kFT;
constexpr int kMaxWords = kFastMaxVocab / 32;  // bitmap words
constexpr int kWordsPer = kMaxWords / kFT;     // bitmap words per thread (rank map build)
constexpr int kMaxWindow = kFT;     // widest window of the count cascade (one bin per thread)
constexpr int kFastHistory = 4096;  // history ids a row of the fast path may have (longer: generic engine)
constexpr int kHistPer = kFastHistory / kFT;
constexpr int kMemPer = kFastMembers / kFT;
constexpr int kSmallK = 64;         // top_k bound of the thread-value path
constexpr int kTvBins = 256;        // bins of the thread-value histogram


typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef short i16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Loads of the row and of the history ids are issued through inline assembly
// and waited for explicitly.  Written as ordinary loads, the compiler moves
// each one down to its first use, after the history work, so that the row
// stream would only start once that work is done; and its own wait for the
// history ids would count the row's loads issued before them.  The waits
// below count loads issued after the one waited for; compiler-issued vector
// memory operations in between only make them wait longer, never shorter.
// The row stream is read once, so its loads carry the non-temporal hint:
// on MI355X the C3 step runs about 1 us faster with it.
__device__ __forceinline__ u32x4 issue_load_b128(const void *p) {
  u32x4 d;
  asm volatile("global_load_dwordx4 %0, %1, off nt" : "=v"(d) : "v"(p));
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
  const uint32_t neg = __builtin_bit_cast(uint32_t, __builtin_bit_cast(i16x2, w) >> (short)15);  // 0xFFFF per negative half
  // w ^ (neg | 0x80008000): truth table of a ^ (b | c) over a = 0xF0, b = 0xCC, c = 0xAA
  return __builtin_amdgcn_bitop3_b32(w, neg, 0x80008000u, (uint8_t)(0xF0 ^ (0xCC | 0xAA)));
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

// LDS arena with phase-dependent views (byte offsets).  The lean pass of
// greedy and small-k rows (lean_row):
//   [0, 32K)      history hash: token + 1 | multiplicity << 18
//   [32K, 42K)    per wave, the chunks it recorded: raw words, chunk index
//   [42K, 44K)    per candidate bin, its lowest index
//   [44K, 59K)    per wave, its candidates (y key << 32 | index); the count
//                 histogram over y keys from the bound; the finishing wave's
//                 group table and index scratch
//   [64K, 68K)    per candidate bin, exp(y - y0) (f64)
// The general pass of every other row (and of a lean row that declines):
//   [0, 10K)      per bitmap word, the number of members before it (history
//                 build); then [0, 57K) SelState: candidate list, sort and
//                 finish scratch
//   [60K, 62K)    window histogram (thread values; count cascade)
//   [62K, 62K+64) counters of the small-k path
//   [64K, 84K)    membership bitmap over the vocab; bits 8 (c & 3) .. 8 (c & 3)
//                 + 7 of word c / 4 are chunk c's members; then the partial
//                 ranks of the small-k finish
//   [84K, 124K)   chunk maxima of the load pass (word w of thread t at
//                 w * kFT + t: slots 2w, 2w + 1)
//   [128K, 152K)  members: token ids, multiplicities, raw key | z key << 16
//   full path: [0, 128K) 65536 16-bit counters; after compaction [128K, 152K)
//   the entries (key << 16 | count) -- the member list waits in registers
//   meanwhile -- and [0, 72K) their prefixes; the ordered search keeps its
//   per-slot / per-thread counts at [0, 4K)
constexpr int kArenaBytes = 152 * 1024;
constexpr int kOffPrefix = 0;
constexpr int kOffWhist = 60 * 1024;
constexpr int kOffCounters = 62 * 1024;
constexpr int kOffBitmap = 64 * 1024;
constexpr int kOffRankScratch = 64 * 1024;
constexpr int kOffCm = 84 * 1024;
constexpr int kOffMembers = 128 * 1024;
constexpr int kOffEntries = 128 * 1024;
constexpr int kOffSlotCnt = 0;
constexpr int kOffTcnt = kMaxSlots * kFW * 4;
constexpr int kLOffHash = 0;             // lean pass: history hash
constexpr int kLHashBits = 13;
constexpr int kLHashSlots = 1 << kLHashBits;
constexpr int kRecSeg = 64;              // chunks a wave records
constexpr int kLOffRecRaw = 32 * 1024;
constexpr int kLOffRecCh = kLOffRecRaw + kFW * kRecSeg * 16;
constexpr int kLOffBinMin = kLOffRecCh + kFW * kRecSeg * 4;  // per candidate bin, its lowest index
constexpr int kOffCand = 44 * 1024;      // candidate list, one segment per wave
constexpr int kCandSeg = 128;            // entries of a wave's segment
constexpr int kOffCandHist = kOffCand + kFW * kCandSeg * 8;
constexpr int kCandBins = 512;           // y keys y0 .. y0 + 510, then one bin for everything above
constexpr int kOffGroups = kOffCandHist + kCandBins * 4;
constexpr int kOffMatch = kOffGroups + 64 * 8;
constexpr int kCtrLeanBad = 6;           // counters() words of the lean pass: a reason to decline,
constexpr int kCtrLeanYmax = 7;          // and the largest listed y key
constexpr int kLOffWbin = 64 * 1024;     // lean pass: exp(y - y0) of each candidate bin (f64)
constexpr int kFinishBins = kCandBins;   // the bins stream_finish scans below the largest key (all)
static_assert(kLOffHash + kLHashSlots * 4 <= kLOffRecRaw && kLOffBinMin + kCandBins * 4 <= kOffCand, "lean views");
static_assert(kOffMatch + kFW * kCandSeg * 4 <= kOffWhist, "candidate views");
static_assert(kFastHistory * 2 <= kLHashSlots && kFastMaxVocab < (1 << 18) && kFastHistory < (1 << 14),
              "hash load and packing");
static_assert(kOffPrefix + kMaxWords * 2 <= kOffWhist, "prefix view");
static_assert((int)sizeof(SelState) <= kOffWhist, "SelState view");
static_assert(kOffWhist + kMaxWindow * 4 <= kOffCounters && kTvBins <= kMaxWindow, "window view");
static_assert(kOffCounters + 64 <= kOffBitmap, "counter view");
static_assert(kOffBitmap + kMaxWords * 4 <= kOffCm, "bitmap view");
static_assert(kOffRankScratch + kFT * 4 <= kOffCm, "rank view");
static_assert(kOffCm + kMaxSlots / 2 * kFT * 4 <= kOffMembers, "chunk maxima view");
static_assert(kOffMembers + kFastMembers * 12 <= kArenaBytes, "member view");
static_assert(kOffEntries + kMaxEntries * 4 <= kArenaBytes, "entries view");
static_assert(kMaxEntries * 12 <= kOffEntries, "prefix view");
static_assert(kOffTcnt + kFT * 4 <= kOffEntries, "ordered search view");
static_assert(kFastMembers % kFT == 0 && kFastHistory % kFT == 0 && kMaxWords % kFT == 0, "per-thread counts");

struct FastShared {
  alignas(16) unsigned char arena[kArenaBytes];
  double dscr[kWaves];
  uint32_t uscr[kWaves];
  uint32_t uscr2[kWaves];
  uint32_t uscr3[kWaves];
  int32_t iscr[kWaves];
  uint32_t chunk_z[8];
  uint32_t bsel[8];
  int32_t lean_l[kFW];      // lean pass: each wave's bound
  uint32_t cand_n[kFW];     // candidates listed by each wave

  __device__ uint32_t *u32(int off) { return (uint32_t *)(arena + off); }
  __device__ uint32_t *m_idx() { return u32(kOffMembers); }
  __device__ uint32_t *m_cnt() { return u32(kOffMembers + kFastMembers * 4); }
  __device__ uint32_t *m_key() { return u32(kOffMembers + kFastMembers * 8); }
  __device__ uint32_t *bitmap() { return u32(kOffBitmap); }
  __device__ uint16_t *prefix() { return (uint16_t *)(arena + kOffPrefix); }
  __device__ uint32_t *whist() { return u32(kOffWhist); }
  __device__ uint32_t *counters() { return u32(kOffCounters); }
  __device__ uint32_t *rank_scratch() { return u32(kOffRankScratch); }
  __device__ SelState &ss() { return *(SelState *)(arena); }
};

// The fast and the generic engine share one LDS allocation.
union FastOrGeneric {
  FastShared f;
  GenericShared g;
};

// Three block-wide maxima with one pair of barriers.
__device__ __forceinline__ void block_max3(uint32_t &a, uint32_t &b, uint32_t &c, FastShared &sh) {
  a = wave_max(a);
  b = wave_max(b);
  c = wave_max(c);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    sh.uscr[threadIdx.x >> 6] = a;
    sh.uscr2[threadIdx.x >> 6] = b;
    sh.uscr3[threadIdx.x >> 6] = c;
  }
  __syncthreads();
  uint32_t ra = sh.uscr[0], rb = sh.uscr2[0], rc = sh.uscr3[0];
#pragma unroll
  for (int i = 1; i < kFW; ++i) {
    ra = max(ra, sh.uscr[i]);
    rb = max(rb, sh.uscr2[i]);
    rc = max(rc, sh.uscr3[i]);
  }
  a = uniform(ra);
  b = uniform(rb);
  c = uniform(rc);
}

// Calls f(Index<s>) for a runtime value s in [B, E) that is uniform across
// the wave, through a tree of scalar branches.
template <int B, int E, class F>
__device__ __forceinline__ void dispatch(int s, F &&f) {
  if constexpr (E - B == 1) {
    f(Index<B>{});
  } else {
    constexpr int M = (B + E) / 2;
    if (s < M)
      dispatch<B, M>(s, f);
    else
      dispatch<M, E>(s, f);
  }
}

// Exclusive position of this lane's n items in a list, with one LDS atomic
// per wave on *counter (which must start at zero for the list).
__device__ __forceinline__ uint32_t wave_reserve(uint32_t n, uint32_t *counter) {
  const uint32_t incl = wave_inclusive<OpSum>(n, 0u);
  uint32_t base = 0u;
  if ((threadIdx.x & 63) == 63 && incl) base = atomicAdd(counter, incl);
  return (uint32_t)__builtin_amdgcn_readlane((int)base, 63) + incl - n;
}

// ---- history members ------------------------------------------------------------

// This thread's history ids (strided by the block), issued as explicit loads;
// positions past the end re-read the first id and are ignored later.  Rows
// without a history load `dummy` instead, so that every row issues the same
// number of loads (the waits count them).
__device__ __forceinline__ void issue_history_ids(uint32_t (&hid)[kHistPer], const lmrs_sample_args &a,
                                                  const RowCfg &c, bool hist, const void *dummy) {
#pragma unroll
  for (int q = 0; q < kHistPer; ++q) {
    const int64_t j = (int64_t)threadIdx.x + (int64_t)q * kFT;
    hid[q] = issue_load_b32(hist ? a.hist_ids + c.h_begin + (j < c.h_len ? j : 0) : (const uint32_t *)dummy);
  }
}

__device__ __forceinline__ bool history_live(int q, uint32_t t, int64_t h_len, int64_t V) {
  return (int64_t)threadIdx.x + (int64_t)q * kFT < h_len && (int64_t)t < V;
}

// Zeroes the small-k counters and histogram bins and, with a history, the
// bitmap words and the multiplicities.  No barrier.
__device__ __forceinline__ void clear_tables(FastShared &sh, bool hist, int nwords) {
  const int tid = threadIdx.x;
  if (tid < 16) sh.counters()[tid] = 0u;
  if (tid < kTvBins) sh.whist()[tid] = 0u;
  if (hist) {
    uint4 *bm = (uint4 *)sh.bitmap();
    for (int i = tid; i < (nwords + 3) / 4; i += kFT) bm[i] = make_uint4(0u, 0u, 0u, 0u);
    uint4 *cnt = (uint4 *)sh.m_cnt();
    for (int i = tid; i < kFastMembers / 4; i += kFT) cnt[i] = make_uint4(0u, 0u, 0u, 0u);
  }
}

// Marks the history ids below V in the bitmap.  Starts and ends with a
// barrier (the bitmap was cleared without one).
__device__ __forceinline__ void mark_history(FastShared &sh, const uint32_t (&hid)[kHistPer], int64_t h_len,
                                             int64_t V) {
  uint32_t *bm = sh.bitmap();
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kHistPer; ++q) {
    const uint32_t t = hid[q];
    if (history_live(q, t, h_len, V)) atomicOr(&bm[t >> 5], 1u << (t & 31u));
  }
  __syncthreads();
}

// Member indices in token order: prefix[w] = the number of members with a
// token below 32 w.  Thread t owns words kWordsPer * t ... kWordsPer * t +
// kWordsPer - 1, so one block scan orders them.  Returns the member count
// (uniform).  Ends with a barrier.
__device__ __forceinline__ uint32_t rank_members(FastShared &sh, int nwords) {
  const int tid = threadIdx.x;
  const uint32_t *bm = sh.bitmap();
  uint16_t *pre = sh.prefix();
  uint32_t n[kWordsPer];
  uint32_t tot = 0u;
#pragma unroll
  for (int i = 0; i < kWordsPer; ++i) {
    const int j = tid * kWordsPer + i;
    n[i] = j < nwords ? (uint32_t)__builtin_popcount(bm[j]) : 0u;
    tot += n[i];
  }
  uint32_t total;
  uint32_t p = block_exclusive_scan<kFW>(tot, sh.uscr, &total);
#pragma unroll
  for (int i = 0; i < kWordsPer; ++i) {
    const int j = tid * kWordsPer + i;
    if (j < nwords) pre[j] = (uint16_t)p;
    p += n[i];
  }
  __syncthreads();
  return total;
}

// Index of member t in token order.
__device__ __forceinline__ uint32_t member_rank(const FastShared &sh, uint32_t t) {
  const uint32_t w = ((const uint32_t *)(sh.arena + kOffBitmap))[t >> 5];
  return (uint32_t)((const uint16_t *)(sh.arena + kOffPrefix))[t >> 5] +
         (uint32_t)__builtin_popcount(w & ((1u << (t & 31u)) - 1u));
}

// Token ids and multiplicities of the members, at their indices.  Ends with
// a barrier.
__device__ __forceinline__ void count_members(FastShared &sh, const uint32_t (&hid)[kHistPer], int64_t h_len,
                                              int64_t V) {
  uint32_t *cnt = sh.m_cnt(), *midx = sh.m_idx();
#pragma unroll
  for (int q = 0; q < kHistPer; ++q) {
    const uint32_t t = hid[q];
    if (history_live(q, t, h_len, V)) {
      const uint32_t m = member_rank(sh, t);
      atomicAdd(&cnt[m], 1u);
      midx[m] = t;  // every copy of a token writes the same id
    }
  }
  __syncthreads();
}

// Raw logits of the members, one 16-bit load each, issued (not waited for)
// as explicit instructions.
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
  const uint32_t *cnt = sh.m_cnt();
  uint32_t zmax = 0u;
#pragma unroll
  for (int q = 0; q < kMemPer; ++q) {
    const uint32_t m = (uint32_t)threadIdx.x + (uint32_t)q * kFT;
    if (m < nmem) {
      const uint32_t zk = bits_key16(penalise_member(mraw[q], cnt[m], c));
      mkey[m] = bits_key16(mraw[q]) | (zk << 16);
      zmax = max(zmax, zk);
      *bad |= is_nan_key16(zk) ? 1u : 0u;
    }
  }
  return zmax;
}

// ---- selection over LDS data ------------------------------------------------------

// Finishes a row from its first k sorted candidates, one per lane of a wave
// (lane i holds entry i, ((~key) << 32 | index)): the min-p cut
// (min_p.rs:45-53), the nucleus cut (top_p.rs:45-58) and softmax_choice
// (strategies/mod.rs:27-55).
template <class TR>
__device__ __forceinline__ void finish_wave(uint64_t g, const RowCfg &c, const lmrs_sample_args &a, int r,
                                            uint32_t k, bool greedy) {
  const uint32_t lane = threadIdx.x & 63u;
  const float y = TR::value(~(uint32_t)(g >> 32));
  if (greedy) {  // Greedy: the first sorted candidate, log_prob 0, no distribution (greedy.rs:22-29)
    if (lane == 0) write_row(a, r, (uint32_t)(g & 0xFFFFFFFFu), 0.0f, y, 0, 1, 1.0);
    return;
  }
  const float M = TR::value(~(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(g >> 32), 0));
  int32_t flags = 0;
  if (c.min_p >= 0.0) {  // the min-p cut (min_p.rs:45-53): a prefix of the k candidates
    const double thr = minp_threshold(M, c);
    const uint32_t kk = (uint32_t)__builtin_popcountll(__ballot(lane < k && minp_keeps(y, thr)));
    if (kk == 0u) {  // softmax_choice of nothing (strategies/mod.rs:28-30)
      if (lane == 0) write_row(a, r, 0u, 0.0f, 0.0f, LMRS_ROW_EMPTY);
      return;
    }
    if (__ballot((lane + 1u == kk || (lane == kk && lane < k)) && minp_near(y, M, thr)))
      flags |= LMRS_ROW_NEAR_BOUNDARY;
    k = kk;
  }
  const bool in = lane < k;
  const double w = in ? exp((double)(y - M)) : 0.0;
  const double incl = wave_inclusive<OpSum>(w, 0.0);
  const double total = lane63(incl);
  if (!(__builtin_isfinite(total) && total > 0.0)) {
    if (lane == 0) write_row(a, r, 0u, 0.0f, 0.0f, LMRS_ROW_DISTRIBUTION);
    return;
  }
  // Cumulative shares use one reciprocal per normaliser: they differ from
  // the reference's quotients by an ulp or two, far inside the 1e-6 margin
  // that flags a row as near a boundary.
  uint32_t keep = k;
  if (c.top_p < 1.0) {
    const double rtot = 1.0 / total;
    const double acc = incl * rtot;
    const uint64_t hit = __ballot(in && acc >= c.top_p);
    if (hit) keep = (uint32_t)__builtin_ctzll(hit) + 1u;
    // nucleus margin at the cut, from the lane of entry keep - 1
    const double prev = (incl - w) * rtot;
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
    const double rkeep = 1.0 / sum_keep;
    const double lo = (incl - w) * rkeep, hi = incl * rkeep;
    double m = 1.0;
    if (pick > 0u && fabs(c.u - lo) < m) m = fabs(c.u - lo);
    if (pick + 1u < keep && fabs(hi - c.u) < m) m = fabs(hi - c.u);
    write_row(a, r, (uint32_t)(g & 0xFFFFFFFFu), (float)log(w * rkeep), y,
              flags | (m < 1e-6 ? LMRS_ROW_NEAR_BOUNDARY : 0), (int32_t)keep, sum_keep);
  }
}

// Chunk maxima of every thread's slots, kept in LDS after the load pass:
// word w of thread t at w * kFT + t holds slots 2w (low half) and 2w + 1.
__device__ __forceinline__ uint32_t cm_word(const FastShared &sh, int w) {
  return ((const uint32_t *)(sh.arena + kOffCm))[w * kFT + threadIdx.x];
}
// The member bits of chunk ch (eight logits: byte ch & 3 of bitmap word ch / 4).
__device__ __forceinline__ uint32_t chunk_m8(const FastShared &sh, uint32_t ch) {
  return (((const uint32_t *)(sh.arena + kOffBitmap))[ch >> 2] >> ((ch & 3u) * 8u)) & 0xFFu;
}

// The K-th largest value among the chunk maxima of the chunks without
// history tokens (hist: a bitmap exists) and the member z keys -- each value stands for a distinct
// element whose z is at least the value -- by a cascade of windows below
// `hi`, each twice as wide as the last.  Returns false (uniformly) when
// fewer than K values exist.
template <int NCH>
__device__ __forceinline__ bool kth_value(FastShared &sh, bool hist, uint32_t nmem, uint32_t K, uint32_t hi,
                                          uint32_t *out) {
  const int tid = threadIdx.x;
  const uint32_t *mkey = sh.m_key();
  uint32_t *wh = sh.whist();
  uint32_t above = 0u, w = 64u;
  for (;;) {
    const uint32_t lo = hi >= w - 1u ? hi - (w - 1u) : 0u;
    const uint32_t nbins = hi - lo + 1u;
    for (uint32_t i = tid; i < nbins; i += kFT) wh[i] = 0u;
    __syncthreads();
#pragma unroll
    for (int s = 0; s < NCH; ++s) {
      const uint32_t v = (cm_word(sh, s >> 1) >> ((s & 1) * 16)) & 0xFFFFu;
      const bool mixed = hist && chunk_m8(sh, (uint32_t)(s * kFT + tid)) != 0u;
      if (!mixed && v >= lo && v <= hi) atomicAdd(&wh[v - lo], 1u);
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

// The K-th largest of the block's thread values (0 = no value; hi and lo are
// the largest and the smallest nonzero one).  First from one-key bins over
// the kTvBins keys below hi; when fewer than K values lie there, from bins
// of 2^s keys over [lo, hi], rounded down to the lower edge of its bin.
// The bins start at zero; every wave scans them itself.  Returns false
// (uniformly) when fewer than K values exist.
__device__ __forceinline__ bool kth_thread(FastShared &sh, uint32_t v, uint32_t hi, uint32_t lo, uint32_t K,
                                           uint32_t *out) {
  uint32_t *wh = sh.whist();
  const uint32_t lane = threadIdx.x & 63u;
  // The bin holding the K-th count (counting from bin 0), its lower edge
  // hi - (((bin + 1) << s) - 1); false when the bins hold fewer than K.
  auto scan = [&](uint32_t s, uint32_t *edge) {
    const uint4 b = ((const uint4 *)wh)[lane];  // bins 4 lane .. 4 lane + 3
    const uint32_t own = b.x + b.y + b.z + b.w;
    const uint32_t incl = wave_inclusive<OpSum>(own, 0u);
    if (lane63(incl) < K) return false;
    const uint32_t l = (uint32_t)__builtin_ctzll(__ballot(incl >= K));
    const uint32_t acc = incl - own;
    uint32_t bin = 4u * lane + 3u;
    if (acc + b.x >= K)
      bin = 4u * lane;
    else if (acc + b.x + b.y >= K)
      bin = 4u * lane + 1u;
    else if (acc + b.x + b.y + b.z >= K)
      bin = 4u * lane + 2u;
    const uint32_t drop = (((uint32_t)__builtin_amdgcn_readlane((int)bin, (int)l) + 1u) << s) - 1u;
    *edge = uniform(hi - lo > drop ? hi - drop : lo);
    return true;
  };
  if (v && hi - v < (uint32_t)kTvBins) atomicAdd(&wh[hi - v], 1u);
  __syncthreads();
  if (scan(0u, out)) return true;
  __syncthreads();  // every wave has read the bins
  if (threadIdx.x < (unsigned)kTvBins) wh[threadIdx.x] = 0u;
  __syncthreads();
  const uint32_t span = hi - lo;
  const uint32_t s = span < (uint32_t)kTvBins ? 0u : 24u - (uint32_t)__builtin_clz(span);
  if (v) atomicAdd(&wh[(hi - v) >> s], 1u);
  __syncthreads();
  return scan(s, out);
}

// Bit e set: key e of the chunk (four packed words) is at least za.
__device__ __forceinline__ uint32_t chunk_ge(const uint4 &w, uint32_t za) {
  const uint32_t x[4] = {w.x, w.y, w.z, w.w};
  uint32_t m = 0u;
#pragma unroll
  for (int e = 0; e < 8; ++e) m |= (((x[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu) >= za ? 1u : 0u) << e;
  return m;
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

// Elements of a chunk (four packed key words) with a key in [lo, hi].
__device__ __forceinline__ uint32_t chunk_matches_keys(const uint4 &w, uint32_t lo, uint32_t hi) {
  const uint32_t x[4] = {w.x, w.y, w.z, w.w};
  uint32_t n = 0u;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t key = (x[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
    n += (key >= lo && key <= hi) ? 1u : 0u;
  }
  return n;
}

// The ordered search for the j-th (1-based) lowest index among elements
// whose z key lies in [lo, hi] (members by their z key).  Index order is
// (slot, thread, element).  The caller has added each wave's count of
// matching raw keys per slot to slot_cnt[s * kFW + wave]; this adds the
// members' net counts, finds the slot holding the j-th match, and, with one
// block scan over that slot's per-thread counts, the chunk and then the
// element.  keys_of(s) returns this thread's chunk of slot s as four packed
// key words (called once, for the chosen slot, by every thread).
template <int NCH, class KeysOf>
__device__ __forceinline__ uint32_t locate_jth(FastShared &sh, int nchunks, uint32_t nmem, uint32_t lo,
                                               uint32_t hi, uint32_t j, KeysOf keys_of) {
  const int tid = threadIdx.x;
  uint32_t *slot_cnt = sh.u32(kOffSlotCnt), *tcnt = sh.u32(kOffTcnt);
  const uint32_t *midx = sh.m_idx(), *mkey = sh.m_key();
  for (uint32_t m = tid; m < nmem; m += kFT) {
    const int dl = member_delta(mkey[m], lo, hi);
    const uint32_t ch = midx[m] >> 3;
    if (dl) atomicAdd(&slot_cnt[(ch / kFT) * kFW + ((ch % kFT) >> 6)], (uint32_t)dl);
  }
  __syncthreads();
  if (tid < NCH) {  // per-slot totals
    uint32_t tot = 0;
    for (int w = 0; w < kFW; ++w) tot += slot_cnt[tid * kFW + w];
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
    sh.bsel[4] = 0u;
  }
  __syncthreads();
  const int sstar = (int)uniform(sh.bsel[0]);
  const uint32_t jr = j - uniform(sh.bsel[1]);
  tcnt[tid] = 0u;
  if (tid < 8) sh.chunk_z[tid] = 0xFFFFFFFFu;
  __syncthreads();
  for (uint32_t m = tid; m < nmem; m += kFT) {  // members of slot sstar, per owner row thread
    const int dl = member_delta(mkey[m], lo, hi);
    const uint32_t ch = midx[m] >> 3;
    if (dl && (int)(ch / kFT) == sstar) atomicAdd(&tcnt[ch % kFT], (uint32_t)dl);
  }
  __syncthreads();
  const int chs = sstar * kFT + tid;
  const uint4 w = keys_of(sstar);
  uint32_t mine = tcnt[tid];
  if (chs < nchunks) mine += chunk_matches_keys(w, lo, hi);
  uint32_t tot;
  const uint32_t excl = block_exclusive_scan<kFW>(mine, sh.uscr, &tot);
  if (excl < jr && jr <= excl + mine) {
    sh.bsel[2] = (uint32_t)chs;  // the chunk
    sh.bsel[3] = jr - excl;      // rank inside it
  }
  __syncthreads();
  const uint32_t cstar = uniform(sh.bsel[2]), need0 = uniform(sh.bsel[3]);
  for (uint32_t m = tid; m < nmem; m += kFT)
    if ((midx[m] >> 3) == cstar) sh.chunk_z[midx[m] & 7u] = mkey[m] >> 16;
  __syncthreads();
  if ((uint32_t)chs == cstar) {  // the owner of the chunk picks the element
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

// The ordered search on a second read of the row (the 65536-bin path, whose
// keys have left the registers): per-slot match counts, G slots in flight.
template <int NCH>
__device__ __forceinline__ uint32_t find_jth_stream(FastShared &sh, const uint4 *src, int nchunks, uint32_t nmem,
                                                    uint32_t lo, uint32_t hi, uint32_t j) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t *slot_cnt = sh.u32(kOffSlotCnt);
  for (int i = tid; i < NCH * kFW; i += kFT) slot_cnt[i] = 0u;
  __syncthreads();
  {
    constexpr int G = 8;  // slots in flight at a time
    const int ft = fresh_tid();
#pragma unroll
    for (int s0 = 0; s0 < NCH; s0 += G) {
      uint4 d[G];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int ch = (s0 + g) * kFT + ft;
        if (s0 + g < NCH) d[g] = *(ch < nchunks ? src + ch : &kNegInfChunk);
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int s = s0 + g;
        if (s < NCH) {
          const uint32_t n = (s * kFT + ft < nchunks) ? chunk_matches(d[g], lo, hi) : 0u;
          const uint32_t t = wave_sum(n);
          if (lane == 0 && t) atomicAdd(&slot_cnt[s * kFW + wave], t);
        }
      }
    }
  }
  return locate_jth<NCH>(sh, nchunks, nmem, lo, hi, j, [&](int s) {
    const int ch = s * kFT + tid;
    const uint4 dd = src[ch < nchunks ? ch : nchunks - 1];
    return make_uint4(key_pair(dd.x), key_pair(dd.y), key_pair(dd.z), key_pair(dd.w));
  });
}

// The ordered search on the keys the load pass left in registers.
template <int NCH>
__device__ __forceinline__ uint32_t find_jth_regs(FastShared &sh, const uint32_t (&k)[NCH][4], int nchunks,
                                                  uint32_t nmem, uint32_t lo, uint32_t hi, uint32_t j) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t *slot_cnt = sh.u32(kOffSlotCnt);
  for (int i = tid; i < NCH * kFW; i += kFT) slot_cnt[i] = 0u;
  __syncthreads();
  const int ft = fresh_tid();
  static_for<0, NCH>([&](auto S) {
    constexpr int s = decltype(S)::value;
    const uint4 w = make_uint4(k[s][0], k[s][1], k[s][2], k[s][3]);
    const uint32_t n = (s * kFT + ft < nchunks) ? chunk_matches_keys(w, lo, hi) : 0u;
    if (__ballot(n != 0u)) {
      const uint32_t t = wave_sum(n);
      if (lane == 0) atomicAdd(&slot_cnt[s * kFW + wave], t);
    }
  });
  return locate_jth<NCH>(sh, nchunks, nmem, lo, hi, j, [&](int sstar) {
    // this thread's chunk of slot sstar, selected from the registers
    uint32_t w0 = 0u, w1 = 0u, w2 = 0u, w3 = 0u;
    static_for<0, NCH>([&](auto S) {
      constexpr int s = decltype(S)::value;
      const bool here = s == sstar;
      w0 = here ? k[s][0] : w0;
      w1 = here ? k[s][1] : w1;
      w2 = here ? k[s][2] : w2;
      w3 = here ? k[s][3] : w3;
    });
    return make_uint4(w0, w1, w2, w3);
  });
}

// The ordered search for a tie group of at most kListCap elements: every
// element whose z key lies in [lo, hi] (members by their z key, the others
// by the raw key in registers) is listed in LDS by its index, and the one
// with exactly j - 1 smaller listed indices is the j-th.  The register pass
// tests a chunk's eight keys with packed 16-bit subtractions and minima; the
// few chunks that hold a match list their elements.  The caller has cleared
// counters()[kCtrList] before its last barrier; every key in [lo, hi] is
// above the padding's -inf (lo > kNegInfKey16).
constexpr int kListCap = kFT;
constexpr int kCtrList = 2;
constexpr int kOffList = 4096;  // inside the SelState region, free after the window
template <int NCH>
__device__ __forceinline__ uint32_t find_jth_list(FastShared &sh, const uint32_t (&k)[NCH][4], uint32_t nmem,
                                                  bool hist, uint32_t lo, uint32_t hi, uint32_t j) {
  const int tid = threadIdx.x;
  uint32_t *list = sh.u32(kOffList), *ctr = &sh.counters()[kCtrList];
  const uint32_t *midx = sh.m_idx(), *mkey = sh.m_key();
  const u16x2 lo2 = {(unsigned short)lo, (unsigned short)lo};
  const uint32_t span = hi - lo;
  auto put = [&](uint32_t idx) {
    const uint32_t p = atomicAdd(ctr, 1u);
    if (p < (uint32_t)kListCap) list[p] = idx;
  };
  const int ft = fresh_tid();
  static_for<0, NCH>([&](auto S) {
    constexpr int s = decltype(S)::value;
    // key - lo per 16-bit half (wrapping: keys below lo become large)
    uint32_t d[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t kq = k[s][q];  // (copied to a scalar before the cast)
      d[q] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, kq) - lo2);
    }
    const uint32_t m = pk_min_u16(pk_min_u16(d[0], d[1]), pk_min_u16(d[2], d[3]));
    if (min(m & 0xFFFFu, m >> 16) <= span) {
      const uint32_t ch = (uint32_t)(s * kFT + ft);
      uint32_t m8 = 0u;
#pragma unroll
      for (int e = 0; e < 8; ++e) m8 |= (((d[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu) <= span ? 1u : 0u) << e;
      if (hist) m8 &= ~chunk_m8(sh, ch);  // members enter by their z key
      for (; m8; m8 &= m8 - 1u) put(ch * 8u + (uint32_t)__builtin_ctz(m8));
    }
  });
  for (uint32_t m = (uint32_t)tid; m < nmem; m += kFT) {
    const uint32_t zk = mkey[m] >> 16;
    if (zk >= lo && zk <= hi) put(midx[m]);
  }
  if (tid == 0) sh.bsel[5] = 0xFFFFFFFFu;  // (no j-th element: the caller falls back)
  __syncthreads();
  const uint32_t n = min(uniform(*ctr), (uint32_t)kListCap);
  if ((uint32_t)tid < n) {
    const uint32_t v = list[tid];
    uint32_t below = 0u;
    for (uint32_t q = 0; q < n; ++q) below += list[q] < v ? 1u : 0u;
    if (below + 1u == j) sh.bsel[5] = v;
  }
  __syncthreads();
  return uniform(sh.bsel[5]);
}

// ---- the full distribution from the window of top keys ----------------------------
//
// A row's mass sits in its top keys: the window pass counts, by LDS atomics
// into one bin per thread, only the elements whose z key lies within kWin
// keys of the largest, and adds every other element's weight exp(y - Mb) in
// f32 (per chunk; f64 across chunks).  That sum enters only the total mass,
// where an error of 3e-7 relative moves the draw's target by that fraction:
// inside the 1e-6 margin that flags a row as near a boundary.  Keys whose y
// lies more than kSkip below a lower bound of the row's maximum are neither
// counted nor summed: at most V e^-kSkip (< 2e-11) of the largest weight, 1,
// which a draw reaches only through the rounding fallback, and then the row
// takes the 65536-bin path.  The cuts and
// the draw then work on the window's entries as the 65536-bin path does on
// all of them.  A row whose top-k, min-p or nucleus cut, or whose target, lies
// below the window's last complete tie group goes to the 65536-bin path.
constexpr int kWin = kFT;                      // window keys: one bin per thread
constexpr float kSkip = 37.0f;                 // e^-37 < 1e-16
constexpr int kOffWinHist = 4096;              // views inside the SelState region, free here
constexpr int kOffWinKey = kOffWinHist + kWin * 4;
constexpr int kOffWinCnt = kOffWinKey + kWin * 4;
constexpr int kOffWinMass = kOffWinCnt + kWin * 4;
constexpr int kOffWinBinMin = kOffWinMass + kWin * 8;  // per bin, its lowest index (compacted rows)
constexpr int kOffWinList = 16 * 1024;          // the listed chunks' keys, then their indices
constexpr int kWinListCap = 2048;
constexpr int kOffWinListCh = kOffWinList + kWinListCap * 16;
static_assert(kOffTcnt + kFT * 4 <= kOffWinHist && kOffWinBinMin + kWin * 4 <= kOffWinList &&
              kOffWinListCh + kWinListCap * 4 <= kOffWhist, "window views");

// Returns false (uniformly, with the registers and the member list intact)
// when the row needs the 65536-bin path.
template <int NCH>
__device__ __forceinline__ bool full_window(FastShared &sh, const lmrs_sample_args &a, int r, const RowCfg &c,
                                            const uint32_t (&k)[NCH][4], int nchunks, uint32_t nmem, bool hist,
                                            uint32_t mx, uint32_t zmem, uint32_t zlow_max, bool k_on) {
  const int tid = threadIdx.x;
  const uint32_t *mkey = sh.m_key(), *midx = sh.m_idx();
  // no element's z key exceeds this: the raw chunk maxima (members' raw keys
  // included) and the members' z keys
  const uint32_t zhb = block_max<kFW>(max(mx, zmem), sh.uscr);
  if (zhb <= kNegInfKey16 || zhb >= 0xFF80u) return false;  // all -inf, or +inf: the 65536-bin path decides
  uint32_t zlo = zhb >= kNegInfKey16 + (uint32_t)kWin ? zhb - (uint32_t)(kWin - 1) : kNegInfKey16 + 1u;
  const float Mb = key16_value(temp_key16(zhb, c));  // at least every element's y
  // zlow_max is an element's z key: its y is at most the row's maximum; the
  // chunks whose largest z key lies below zskip hold only weights below e^-kSkip
  const float ys = key16_value(temp_key16(zlow_max, c)) - kSkip;
  // the lowest key whose y reaches ys (zlow_max's does): a search over the
  // lanes, each round testing 64 keys spread over the range left (at most
  // four rounds over the 16-bit keys)
  uint32_t zskip = zlow_max;
  {
    const uint32_t lane = (uint32_t)tid & 63u;
    uint32_t lo = kNegInfKey16;  // the answer lies in [lo, zskip]
    while (lo < zskip) {
      const uint32_t step = (zskip - lo + 62u) / 63u;  // lane 63 tests zskip itself
      const uint32_t kk = min(lo + lane * step, zskip);
      const uint64_t ok = __ballot(key16_value(temp_key16(kk, c)) >= ys);
      const uint32_t f = (uint32_t)__builtin_ctzll(ok);  // ok has lane 63
      const uint32_t hi = min(lo + f * step, zskip);
      lo = f ? lo + (f - 1u) * step + 1u : lo;
      zskip = hi;
    }
  }
  zlo = max(zlo, zskip);  // keys below zskip are neither counted nor summed
  // every element below the window weighs less than e^-kSkip: a cut that
  // falls there changes the kept mass by under 2e-11 of it, and the draw's
  // target can reach those elements only through the rounding fallback
  const bool tail_negligible = zlo == zskip;
  // weight exp(y - Mb) as exp2(y log2(e) - Mb log2(e)), one multiply-add
  const float l2e = 1.4426950408889634f, mb2 = Mb * l2e;
  uint32_t *wh = sh.u32(kOffWinHist), *wmin = sh.u32(kOffWinBinMin);
  wh[tid] = 0u;
  wmin[tid] = 0xFFFFFFFFu;
  bool track_min = false;  // (uniform) the bins' lowest indices are kept: the compacted pass
  // One chunk's window counts (by LDS atomics) and the weight sum of its
  // elements below the window.
  auto window_chunk = [&](const uint4 &w, uint32_t ch) {
    const uint32_t x[4] = {w.x, w.y, w.z, w.w};
    const uint32_t m8 = hist ? chunk_m8(sh, ch) : 0u;  // members enter by their z key
    float acc = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t key = (x[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
      const bool mem = (m8 >> e) & 1u;
      if (!mem && key >= zlo) {
        atomicAdd(&wh[zhb - key], 1u);
        if (track_min) atomicMin(&wmin[zhb - key], ch * 8u + (uint32_t)e);
      }
      const float wt = __builtin_amdgcn_exp2f(__builtin_fmaf(key16_value(temp_key16(key, c)), l2e, -mb2));
      acc += (mem || key >= zlo || key < zskip) ? 0.0f : wt;
    }
    return acc;
  };
  // The chunks with a key at or above zskip (the others are skipped).  When
  // the window reaches zskip (heavy-tailed rows) they are usually few: then
  // they are listed in LDS first, so that each thread takes about one;
  // otherwise every thread works through its own slots.  The scan's
  // barriers also order the histogram's clear.
  const int ft = fresh_tid();
  uint64_t live = 0u;
  static_for<0, NCH>([&](auto S) {
    constexpr int s = decltype(S)::value;
    live |= (uint64_t)((s * kFT + ft < nchunks && chunk_max(k[s]) >= zskip) ? 1u : 0u) << s;
  });
  uint32_t nlive = 0xFFFFFFFFu, lpos = 0u;
  if (tail_negligible)
    lpos = block_exclusive_scan<kFW>((uint32_t)__builtin_popcountll(live), sh.uscr, &nlive);
  else
    __syncthreads();
  double below = 0.0;
  if (nlive <= (uint32_t)kWinListCap) {
    track_min = true;
    uint4 *lk = (uint4 *)sh.u32(kOffWinList);
    uint32_t *lc = sh.u32(kOffWinListCh), p = lpos;
    static_for<0, NCH>([&](auto S) {
      constexpr int s = decltype(S)::value;
      if ((live >> s) & 1u) {
        lk[p] = make_uint4(k[s][0], k[s][1], k[s][2], k[s][3]);
        lc[p] = (uint32_t)(s * kFT + ft);
        ++p;
      }
    });
    __syncthreads();
    for (uint32_t i = (uint32_t)tid; i < nlive; i += kFT) below += (double)window_chunk(lk[i], lc[i]);
  } else {
    static_for<0, NCH>([&](auto S) {
      constexpr int s = decltype(S)::value;
      if ((live >> s) & 1u)
        below += (double)window_chunk(make_uint4(k[s][0], k[s][1], k[s][2], k[s][3]), (uint32_t)(s * kFT + ft));
    });
  }
  for (uint32_t m = tid; m < nmem; m += kFT) {
    const uint32_t zk = mkey[m] >> 16;
    if (zk >= zlo) {
      atomicAdd(&wh[zhb - zk], 1u);
      if (track_min) atomicMin(&wmin[zhb - zk], midx[m]);
    } else if (zk >= zskip)
      below += (double)__builtin_amdgcn_exp2f(__builtin_fmaf(key16_value(temp_key16(zk, c)), l2e, -mb2));
  }
  below = block_sum<kFW>(below, sh.dscr);  // (its barriers order the histogram too)
  // entries: thread t holds bin t, key zhb - t, in descending key order
  const uint32_t cn = wh[tid];
  uint32_t nbu;
  const uint32_t pos = block_exclusive_scan<kFW>(cn != 0u ? 1u : 0u, sh.uscr, &nbu);
  uint32_t *ekey = sh.u32(kOffWinKey), *ecnt = sh.u32(kOffWinCnt);
  if (cn) {
    ekey[pos] = zhb - (uint32_t)tid;
    ecnt[pos] = cn;
  }
  __syncthreads();
  const int nb = (int)nbu;
  if (nb == 0) return false;
  auto ykey_of = [&](int e) { return temp_key16(ekey[e], c); };
  const float M = key16_value(ykey_of(0));
  if (!((double)Mb - (double)M <= 40.0)) return false;  // the f32 weights below would lose their range
  auto weight_of = [&](int e) { return exp((double)(key16_value(ykey_of(e)) - M)); };
  // inclusive count and mass prefixes, entry e at thread e
  uint32_t *cincl = ecnt;  // (in place: each thread reads its count first)
  double *mincl = (double *)sh.u32(kOffWinMass);
  const uint32_t ce = tid < nb ? ecnt[tid] : 0u;
  const double me = tid < nb ? (double)ce * weight_of(tid) : 0.0;
  uint32_t ctot;
  double mtot;
  const uint32_t cex = block_exclusive_scan<kFW>(ce, sh.uscr, &ctot);
  const double mex = block_exclusive_scan<kFW>(me, sh.dscr, &mtot);
  if (tid < nb) {
    cincl[tid] = cex + ce;
    mincl[tid] = mex + me;
  }
  __syncthreads();
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
  auto cnt_of = [&](int e) { return cincl[e] - (e > 0 ? cincl[e - 1] : 0u); };
  auto cnt_excl = [&](int e) { return e > 0 ? cincl[e - 1] : 0u; };
  auto mass_excl = [&](int e) { return e > 0 ? mincl[e - 1] : 0.0; };
  // the last tie group continues below the window when key zlo - 1 has its
  // y: entries [0, hg) are complete
  const int hg = temp_key16(zlo - 1u, c) == ykey_of(nb - 1) ? group_head(nb - 1) : nb;
  if (hg == 0) return false;
  auto first_mass = [&](double target, int last) {  // first entry <= last reaching target; -1 if none
    int f = 0x7FFFFFFF;
    if (tid <= last && mincl[tid] >= target) f = tid;
    f = block_min<kFW>(f, sh.iscr);
    return f == 0x7FFFFFFF ? -1 : f;
  };
  const double total = mtot + below * exp((double)Mb - (double)M);
  // candidates.  last_h: head of the last kept tie group, or nb when the
  // kept set runs below the window (then no window group is cut short)
  int last_e = hg - 1, last_h = nb;
  uint32_t last_keep = 0u;
  double cand_mass = total;
  // the kept count (every element when no cut applies; -1 where a cut falls
  // among the negligible elements, whose keys the window does not count)
  int64_t kept_n = a.vocab;
  if (k_on) {
    kept_n = c.top_k;  // top-k keeps k tokens (k < V)
    int f = 0x7FFFFFFF;
    if (tid < hg && cincl[tid] >= (uint32_t)c.top_k) f = tid;
    f = block_min<kFW>(f, sh.iscr);
    if (f != 0x7FFFFFFF) {
      last_h = group_head(f);
      last_e = group_tail(f);
      last_keep = (uint32_t)c.top_k - cnt_excl(last_h);
      cand_mass = mass_excl(last_h) + (double)last_keep * weight_of(last_h);
    } else if (!tail_negligible) {
      return false;  // the k-th token lies below the window
    }
  }
  int32_t flags = 0;
  if (c.min_p >= 0.0) {  // the min-p cut (min_p.rs:45-53)
    const double thr = minp_threshold(M, c);
    if (!(thr == thr)) {  // NaN threshold: softmax_choice of nothing (strategies/mod.rs:28-30)
      if (tid == 0) write_row(a, r, 0u, 0.0f, 0.0f, LMRS_ROW_EMPTY);
      return true;
    }
    const uint32_t ymp = minp_low_key(kNegInfKey16, ykey_of(0), thr, [](uint32_t kk) { return key16_value(kk); });
    int fm = 0x7FFFFFFF;
    if (tid < nb && ykey_of(tid) < ymp) fm = tid;
    fm = block_min<kFW>(fm, sh.iscr);
    if (fm == 0x7FFFFFFF) fm = nb;
    if (fm == 0) {  // not reached: the maximum always passes a non-NaN threshold
      if (tid == 0) write_row(a, r, 0u, 0.0f, 0.0f, LMRS_ROW_EMPTY);
      return true;
    }
    if (fm - 1 < last_h) {  // the cut ends above the top-k set's last tie group
      // ... known when a window entry fails the cut and every kept entry is
      // complete, or when the cut falls among the negligible elements
      if (fm < nb) {
        if (fm > hg) return false;
        last_e = fm - 1;
        last_h = group_head(last_e);
        last_keep = cnt_excl(last_e) + cnt_of(last_e) - cnt_excl(last_h);
        cand_mass = mincl[last_e];
        kept_n = cincl[last_e];
      } else if (!tail_negligible) {
        return false;
      } else {
        kept_n = -1;
      }
    }
    if (minp_near(key16_value(ymp), M, thr) || (ymp > kNegInfKey16 && minp_near(key16_value(ymp - 1u), M, thr)))
      flags |= LMRS_ROW_NEAR_BOUNDARY;
  }
  if (!(__builtin_isfinite(cand_mass) && cand_mass > 0.0)) {  // (strategies/mod.rs:39-43)
    if (tid == 0) write_row(a, r, 0u, 0.0f, 0.0f, LMRS_ROW_DISTRIBUTION);
    return true;
  }
  double kept_mass = cand_mass;
  if (c.top_p < 1.0) {  // nucleus cut (top_p.rs:45-58) over the candidates
    const double tp = c.top_p * cand_mass;
    const int f = first_mass(tp, last_e);
    if (f < 0) return false;  // the nucleus runs below the window
    const int h = group_head(f), t = group_tail(f);
    const double wg = weight_of(h), mx2 = mass_excl(h);
    const uint32_t gmax = (h == last_h) ? last_keep : cincl[t] - cnt_excl(h);
    double jj = ceil((tp - mx2) / wg);
    if (!(jj >= 1.0)) jj = 1.0;
    if (jj > (double)gmax) jj = (double)gmax;
    const uint32_t jp = (uint32_t)jj;
    kept_mass = mx2 + (double)jp * wg;
    kept_n = (int64_t)cnt_excl(h) + jp;
    const double acc = kept_mass / cand_mass, prev = (kept_mass - wg) / cand_mass;
    double m = c.top_p - prev;
    if (acc - c.top_p < m) m = acc - c.top_p;
    if (m < 1e-6) flags |= LMRS_ROW_NEAR_BOUNDARY;
    last_h = h;
    last_e = t;
    last_keep = jp;
  }
  // the draw (softmax_choice, strategies/mod.rs:44-54)
  const double target = c.u * kept_mass;
  const int f = first_mass(target, last_e);
  if (f < 0) return false;  // below the window (or the rounding fallback: the 65536-bin path has it)
  const int h = group_head(f), tl = group_tail(f);
  const double mx2 = mass_excl(h), wg = weight_of(h);
  const uint32_t gmax = (h == last_h) ? last_keep : cincl[tl] - cnt_excl(h);
  double jj = ceil((target - mx2) / wg);
  if (!(jj >= 1.0)) jj = 1.0;
  if (jj > (double)gmax) jj = (double)gmax;
  const uint32_t jt = (uint32_t)jj;
  const uint32_t zhi = uniform(ekey[h]), zlo2 = uniform(ekey[tl]);
  const uint32_t gtot = uniform(cincl[tl] - cnt_excl(h));  // the group's elements
  const float yv = key16_value(ykey_of(h));
  const bool first_tok = (h == 0 && jt == 1u), last_tok = (h == last_h && jt == gmax);
  // the first token of its tie group: the lowest index over the group's bins
  uint32_t token = ~0u;
  if (track_min && jt == 1u) {
    for (int e = h; e <= tl; ++e) token = min(token, wmin[zhb - ekey[e]]);
    token = uniform(token);
  }
  if (tid == 0) sh.counters()[kCtrList] = 0u;
  __syncthreads();  // the window views are dead
  if (token == ~0u)
    token = gtot <= (uint32_t)kListCap ? find_jth_list<NCH>(sh, k, nmem, hist, zlo2, zhi, jt) : ~0u;
  if (token == ~0u) token = find_jth_regs<NCH>(sh, k, nchunks, nmem, zlo2, zhi, jt);
  if (tid == 0) {
    const double lo_c = (mx2 + (double)(jt - 1u) * wg) / kept_mass, hi_c = lo_c + wg / kept_mass;
    double m = 1.0;
    if (!first_tok && fabs(c.u - lo_c) < m) m = fabs(c.u - lo_c);
    if (!last_tok && fabs(hi_c - c.u) < m) m = fabs(hi_c - c.u);
    write_row(a, r, token, (float)log(wg / kept_mass), yv, flags | (m < 1e-6 ? LMRS_ROW_NEAR_BOUNDARY : 0),
              (int32_t)kept_n, kept_mass);
  }
  return true;
}

// The j-th (1-based) lowest index among the candidates whose y key is yk
// (one wave; j at most their number).  Wave w listed cand_n[w] candidates
// at entries w kCandSeg ... of the list.
__device__ __forceinline__ uint32_t stream_nth_index(FastShared &sh, uint32_t yk, uint32_t j) {
  const uint32_t lane = threadIdx.x & 63u;
  uint32_t cn[kFW];
#pragma unroll
  for (int w = 0; w < kFW; ++w) cn[w] = uniform(sh.cand_n[w]);
  const uint64_t *cand = (const uint64_t *)sh.u32(kOffCand);
  uint32_t *mt = sh.u32(kOffMatch);
  uint32_t m = 0u;
#pragma unroll
  for (int w = 0; w < kFW; ++w) {
    for (uint32_t b = 0u; b < cn[w]; b += 64u) {
      const uint32_t i = b + lane;
      const uint64_t e = i < cn[w] ? cand[w * kCandSeg + i] : ~0ull;
      const bool hit = i < cn[w] && (uint32_t)(e >> 32) == yk;
      const uint64_t mask = __ballot(hit);
      if (hit)
        mt[m + __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u))] =
            (uint32_t)e;
      m += (uint32_t)__builtin_popcountll(mask);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");  // the wave's LDS writes before its reads
  if (m <= 64u) {  // rank among at most 64, one per lane
    const uint32_t v = lane < m ? mt[lane] : 0xFFFFFFFFu;
    uint32_t rank = 0u;
    for (uint32_t q = 0u; q < m; ++q) rank += (uint32_t)__builtin_amdgcn_readlane((int)v, (int)q) < v ? 1u : 0u;
    const uint64_t pick = __ballot(lane < m && rank + 1u == j);
    return (uint32_t)__builtin_amdgcn_readlane((int)v, pick ? (int)__builtin_ctzll(pick) : 0);
  }
  // the smallest x with at least j indices <= x, one bit at a time
  uint32_t res = 0u;
  for (int bit = 17; bit >= 0; --bit) {
    const uint32_t t = res | (1u << bit);
    uint32_t below = 0u;
    for (uint32_t q = lane; q < m; q += 64u) below += mt[q] < t ? 1u : 0u;
    if (wave_sum(below) < j) res = t;
  }
  return res;
}

// Finishes a greedy or small-k row from its listed candidates: every element
// whose y key is at least y0, in per-wave segments (cand_n), with their y
// keys counted in the histogram from y0, the lowest index of each bin in
// binmin, the largest key in counters()[kCtrLeanYmax] and each bin's weight
// exp(y - y0) in wbin (every wave enters, after a barrier).  Every wave reads
// the bins below the largest key, 64 at a time, one per lane, and finds the
// group (y key) of the K-th token; one wave finishes from the groups in
// descending y:
// weights times counts, the min-p and nucleus cuts and the draw
// (softmax_choice, strategies/mod.rs:27-55), and the chosen token, the j-th
// lowest index among the candidates of its group -- the reference's order
// (value descending, index ascending, strategies/mod.rs:21-25), since the
// tokens of a group share their weight.  The weights are the reference's
// exp(y - max) times exp(max - y0): the cuts and the draw compare ratios of
// sums, which that common factor leaves as they are (up to the last bit).
// Returns false (uniformly, with nothing written) when a flag is set (a NaN,
// an overflowed segment), fewer than K tokens lie in the 256 bins below the
// largest key, the
// largest key lies above the bins or more than 700 above y0 in value (its
// weight would near the f64 range; the general pass also takes the rows the
// reference rejects for a non-finite maximum), or the K-th
// token is in the lowest listed group while that group may continue below
// the listed keys (tie_below).
__device__ __forceinline__ bool stream_finish(FastShared &sh, const lmrs_sample_args &a, int r, const RowCfg &c,
                                              uint32_t K, uint32_t y0, bool tie_below) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t ymax = uniform(sh.counters()[kCtrLeanYmax]);
  if (uniform(sh.counters()[kCtrLeanBad]) != 0u || ymax < y0) return false;
  const uint32_t bmax = ymax - y0;
  if (bmax >= (uint32_t)kCandBins - 1u) return false;  // the largest candidates lie above the bins
  // weights up to e^700 keep every sum of at most kCandCap of them finite
  if (!(key16_value(ymax) - key16_value(y0) <= 700.0f)) return false;
  // Rounds of 64 bins in descending y keys (lane l of round e: bin bmax - l -
  // 64 e) until the count reaches K; the non-empty bins down to the K-th
  // token's go, in order, to lanes 0 .. G - 1 (G <= K <= 64: one token each
  // at least) as bin << 20 | count.
  const uint32_t *hb = sh.u32(kOffCandHist);
  uint32_t base = 0u, G = 0u, keep_k = 0u, packed = 0u;
  bool found = false;
  // (all the candidate bins: with 256, heavy-tailed rows whose K-th token lay
  // further below the maximum declined and were read again)
  static_assert(kFinishBins == 8 * 64, "eight rounds of 64 bins");
  for (int e = 0; e < kFinishBins / 64 && !found; ++e) {
    const int bl = (int)bmax - (int)lane - 64 * e;
    const uint32_t cnt = bl >= 0 ? hb[bl] : 0u;
    const uint32_t incl = wave_inclusive<OpSum>(cnt, 0u) + base;
    const uint64_t reach = __ballot(incl >= K);
    const uint32_t lim = reach ? (uint32_t)__builtin_ctzll(reach) : 63u;  // lanes within the cut
    const bool ne = cnt != 0u && lane <= lim;
    const uint64_t nzm = __ballot(ne), zm = ~nzm;
    const uint32_t n = (uint32_t)__builtin_popcountll(nzm);
    // a permutation of the lanes: the bins to G .. G + n - 1, the others around them
    const uint32_t d = __builtin_amdgcn_mbcnt_hi((uint32_t)(zm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)zm, 0u));
    const uint32_t dest = ne ? G + __builtin_amdgcn_mbcnt_hi((uint32_t)(nzm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)nzm, 0u))
                             : (d < G ? d : d + n);
    packed |= (uint32_t)__builtin_amdgcn_ds_permute((int)(dest * 4u), (int)(ne ? (((uint32_t)bl << 20) | cnt) : 0u));
    G += n;
    if (reach) {
      found = true;
      keep_k = K - ((uint32_t)__builtin_amdgcn_readlane((int)incl, (int)lim) -
                    (uint32_t)__builtin_amdgcn_readlane((int)cnt, (int)lim));
      // the K-th token in the lowest listed bin, which may continue below za
      if (tie_below && bmax == lim + 64u * (uint32_t)e) return false;
    } else {
      base = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
    }
  }
  if (!found) return false;
  if (threadIdx.x >= 64u) return true;  // one wave finishes the row
  const bool in = lane < G;
  const uint32_t gb = in ? packed >> 20 : 0u;                       // the group's bin (y key - y0)
  const uint32_t yk = y0 + gb;
  const uint32_t gcnt = lane + 1u == G ? keep_k : (packed & 0xFFFFFu);  // the K-th token's group keeps keep_k
  const uint32_t *binmin = sh.u32(kLOffBinMin);
  const float M = key16_value(ymax);
  if (c.greedy) {  // Greedy (greedy.rs:22-29): the lowest index at the maximum, log_prob 0
    const uint32_t tok = uniform(binmin[bmax]);
    if (lane == 0u) write_row(a, r, tok, 0.0f, M, LMRS_ROW_OK, 1, 1.0);
    return true;
  }
  const double w = in ? ((const double *)sh.u32(kLOffWbin))[gb] : 0.0;  // exp(y - y0) per token
  const bool dist = a.kept_count || a.kept_mass;  // the post-filter distribution is asked for
  const uint32_t cnt_incl = dist ? wave_inclusive<OpSum>(in ? gcnt : 0u, 0u) : 0u;  // tokens of groups 0 .. lane
  const double rw = in ? 1.0 / w : 0.0;
  const double incm = wave_inclusive<OpSum>(w * (double)gcnt, 0.0);
  const double excl = incm - w * (double)gcnt;
  auto at = [](double v, uint32_t l) {
    const uint64_t u = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, (int)l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), (int)l);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
  };
  uint32_t last = G - 1u, last_keep = keep_k;  // the last kept group, and its kept tokens
  double cand_mass = at(incm, last);
  int32_t flags = 0;
  if (c.min_p >= 0.0) {  // the min-p cut (min_p.rs:45-53): a prefix of the groups
    const double thr = minp_threshold(M, c);
    if (!(thr == thr)) {  // NaN threshold: softmax_choice of nothing (strategies/mod.rs:28-30)
      if (lane == 0u) write_row(a, r, 0u, 0.0f, 0.0f, LMRS_ROW_EMPTY);
      return true;
    }
    const uint32_t ymp = minp_low_key(kNegInfKey16, ymax, thr, [](uint32_t kk) { return key16_value(kk); });
    const uint32_t gm = (uint32_t)__builtin_popcountll(__ballot(in && yk >= ymp));
    if (gm == 0u) {  // not reached: the maximum passes every non-NaN threshold
      if (lane == 0u) write_row(a, r, 0u, 0.0f, 0.0f, LMRS_ROW_EMPTY);
      return true;
    }
    if (gm < G) {  // the cut ends above the K-th token's group: group gm - 1 is kept whole
      last = gm - 1u;
      last_keep = (uint32_t)__builtin_amdgcn_readlane((int)gcnt, (int)last);
      cand_mass = at(incm, last);
    }
    if (minp_near(key16_value(ymp), M, thr) || (ymp > kNegInfKey16 && minp_near(key16_value(ymp - 1u), M, thr)))
      flags |= LMRS_ROW_NEAR_BOUNDARY;
  }
  if (!(__builtin_isfinite(cand_mass) && cand_mass > 0.0)) {  // (strategies/mod.rs:39-43)
    if (lane == 0u) write_row(a, r, 0u, 0.0f, 0.0f, LMRS_ROW_DISTRIBUTION);
    return true;
  }
  // inclusive mass of each group, the last one cut to its kept tokens
  auto cum_of = [&](uint32_t lst, uint32_t lkeep) { return lane < lst ? incm : excl + (double)lkeep * w; };
  double kept = cand_mass;
  if (c.top_p < 1.0) {  // nucleus cut (top_p.rs:45-58) over the candidates
    const double tp = c.top_p * cand_mass;
    const uint64_t hit = __ballot(lane <= last && cum_of(last, last_keep) >= tp);
    const uint32_t f = hit ? (uint32_t)__builtin_ctzll(hit) : last;
    const double wf = at(w, f), ef = at(excl, f);
    const uint32_t gmax = f == last ? last_keep : (uint32_t)__builtin_amdgcn_readlane((int)gcnt, (int)f);
    double jj = ceil((tp - ef) * at(rw, f));
    if (!(jj >= 1.0)) jj = 1.0;
    if (jj > (double)gmax) jj = (double)gmax;
    const uint32_t jp = (uint32_t)jj;
    kept = ef + (double)jp * wf;
    const double rc = 1.0 / cand_mass, accp = kept * rc, prev = (kept - wf) * rc;
    double m = c.top_p - prev;
    if (accp - c.top_p < m) m = accp - c.top_p;
    if (m < 1e-6) flags |= LMRS_ROW_NEAR_BOUNDARY;
    last = f;
    last_keep = jp;
  }
  // the draw (softmax_choice, strategies/mod.rs:44-54)
  const double target = c.u * kept;
  const uint64_t hit = __ballot(lane <= last && cum_of(last, last_keep) >= target);
  const uint32_t f = hit ? (uint32_t)__builtin_ctzll(hit) : last;  // fallback: the last kept token
  const double wf = at(w, f), ef = at(excl, f);
  const uint32_t gmax = f == last ? last_keep : (uint32_t)__builtin_amdgcn_readlane((int)gcnt, (int)f);
  double jj = hit ? ceil((target - ef) * at(rw, f)) : (double)gmax;
  if (!(jj >= 1.0)) jj = 1.0;
  if (jj > (double)gmax) jj = (double)gmax;
  const uint32_t jt = (uint32_t)jj;
  const uint32_t gbf = (uint32_t)__builtin_amdgcn_readlane((int)gb, (int)f), ykf = y0 + gbf;
  const uint32_t tok = jt == 1u ? uniform(binmin[gbf]) : stream_nth_index(sh, ykf, jt);
  // the kept set: groups before `last` whole, then last_keep tokens (the
  // prefix sum runs with every lane active, outside the branch below); its
  // mass against the row's maximum, group 0's weight exp(M - y0)
  const uint32_t before = dist && last > 0u ? (uint32_t)__builtin_amdgcn_readlane((int)cnt_incl, (int)(last - 1u)) : 0u;
  const double w0 = dist ? at(w, 0u) : 1.0;
  if (lane == 0u) {
    // ln(w / kept) = (y - y0) - ln(kept), the difference exact in f32; ln(kept)
    // from log2 of its mantissa in [0.5, 1) (within 1e-7) and its exponent
    const float yv = key16_value(ykf);
    int ek;
    const double mk = frexp(kept, &ek);
    const double lnk = ((double)__builtin_amdgcn_logf((float)mk) + (double)ek) * 0.6931471805599453;
    const double rk = 1.0 / kept;
    const double lo_c = (ef + (double)(jt - 1u) * wf) * rk, hi_c = lo_c + wf * rk;
    double m = 1.0;
    if (!(f == 0u && jt == 1u) && fabs(c.u - lo_c) < m) m = fabs(c.u - lo_c);
    if (!(f == last && jt == gmax) && fabs(hi_c - c.u) < m) m = fabs(hi_c - c.u);
    if (!hit) m = 0.0;
    write_row(a, r, tok, (float)((double)(yv - key16_value(y0)) - lnk), yv,
              flags | (m < 1e-6 ? LMRS_ROW_NEAR_BOUNDARY : 0), (int32_t)(before + last_keep), kept / w0);
  }
  return true;
}

// ---- the lean pass of greedy and small-k rows ----------------------------------------
//
// A row that keeps at most kSmallK tokens by top-k (greedy included), whose
// penalties can only lower a history token's logit, is selected while it
// streams in, with as few instructions per slot as possible (each one runs
// on eight waves that share four SIMDs):
//   * per slot, the chunk's maximum as signed 16-bit integers of the raw
//     bf16 patterns -- the true maximum whenever it is not negative -- and
//     the unsigned maximum, which exposes a negative NaN;
//   * from slot kHashFrom the history ids go into an LDS hash (token ->
//     multiplicity), one a slot, while the row streams in;
//   * at slot kBoundAt (half the row; from slot kDeepAt every later slot is
//     requested) a bound: each wave takes the ceil(K/8)-th largest of its threads'
//     running maxima, and the row's bound za is the smallest of the eight.
//     Every chunk whose maximum reaches za is recorded (raw words and index)
//     in its wave's LDS segment, those of the slots already in registers at
//     once, the later ones as they land;
//   * after the last slot each wave turns its own records into candidates:
//     elements with z >= za (a history token by its penalised z, which is
//     never above its raw logit here), each listed as (y key, index) and
//     counted in a histogram over y keys, and its index in the lowest index
//     of its bin; one barrier, then stream_finish.
// Nothing here has to be a proof: za stands for the values of real elements
// only when they are not negative, and any number of history tokens may sit
// among the maxima.  What matters is that every element with z >= za is
// listed: if at least K are, the K largest by (y, index) are among them, and
// stream_finish checks that count -- and that the K-th is not in the lowest
// listed group when under temperature that group also holds keys below za.  A row that has fewer, a negative bound,
// a NaN, or more records or candidates than a segment holds declines, and
// the general pass takes it from the registers.

// Signed maximum of the eight bf16 patterns of a chunk (as int16): the
// largest value when any value is >= +0.0.  The words are copied out first:
// a __builtin_bit_cast of an element of a vector reference (w[1]) is
// compiled here as a cast of the vector's first element.
__device__ __forceinline__ int32_t chunk_smax(const u32x4 &w) {
  const uint32_t w0 = w[0], w1 = w[1], w2 = w[2], w3 = w[3];
  const i16x2 a = __builtin_elementwise_max(__builtin_bit_cast(i16x2, w0), __builtin_bit_cast(i16x2, w1));
  const i16x2 b = __builtin_elementwise_max(__builtin_bit_cast(i16x2, w2), __builtin_bit_cast(i16x2, w3));
  const i16x2 m = __builtin_elementwise_max(a, b);
  return max((int32_t)m.x, (int32_t)m.y);
}

// Unsigned maxima of the bf16 patterns (two halves): a negative NaN is a
// pattern above 0xFF80.
__device__ __forceinline__ uint32_t chunk_umax(const u32x4 &w) {
  return pk_max_u16(pk_max_u16(w[0], w[1]), pk_max_u16(w[2], w[3]));
}

__device__ __forceinline__ uint32_t lean_hash_slot(uint32_t t) { return (t * 2654435761u) >> (32 - kLHashBits); }

// Adds one occurrence of history token t (t < V) to the hash.
__device__ __forceinline__ void lean_hash_add(uint32_t *h, uint32_t t) {
  const uint32_t key = t + 1u;
  for (uint32_t s = lean_hash_slot(t);; s = (s + 1u) & (kLHashSlots - 1)) {  // ends: at most half full
    const uint32_t old = atomicCAS(&h[s], 0u, key | (1u << 18));
    if (old == 0u) return;
    if ((old & 0x3FFFFu) == key) {
      atomicAdd(&h[s], 1u << 18);
      return;
    }
  }
}

// Multiplicity of token t in the history (0: not a history token).
__device__ __forceinline__ uint32_t lean_hash_count(const uint32_t *h, uint32_t t) {
  const uint32_t key = t + 1u;
  for (uint32_t s = lean_hash_slot(t);; s = (s + 1u) & (kLHashSlots - 1)) {
    const uint32_t v = h[s];
    if (v == 0u) return 0u;
    if ((v & 0x3FFFFu) == key) return v >> 18;
  }
}

// Whether a row's penalties can only lower a history token's logit (then
// z <= raw for every element): repetition >= 1, presence and frequency >= 0.
__device__ __forceinline__ bool penalties_lower(const RowCfg &c) {
  return (!c.rep_on || c.nf >= 1.0f) && (!c.pres_on || (c.presence >= 0.0f && c.frequency >= 0.0f));
}

// The lean pass of one row.  On entry slots 0 .. kPre - 1 and the history
// ids are requested; returns true when the row is written, false (uniformly)
// when the general pass must take it, with every slot waited for in kv (raw
// patterns) and the history ids in hid.
template <int NCH, int kPre>
__device__ __forceinline__ bool lean_row(FastShared &sh, const lmrs_sample_args &a, int r, const RowCfg &c,
                                         u32x4 (&kv)[NCH], uint32_t (&hid)[kHistPer], bool hist, const uint4 *src,
                                         int nchunks) {
  const int tid = threadIdx.x;
  const uint32_t lane = (uint32_t)tid & 63u;
  const int wave = tid >> 6;
  const int64_t V = a.vocab;
  constexpr int kEarly = NCH / 4;      // slots in flight ahead of the one being processed
  constexpr int kBoundAt = NCH / 2;    // the bound is taken before this slot is waited for
  constexpr int kDeepAt = NCH / 2;     // from this slot on, every slot of the row is requested
  constexpr int kHashFrom = kPre + 1;  // from this slot, kHashPer history ids a slot enter the hash
  constexpr int kHashPer = (kHistPer + (NCH - kHashFrom) - 1) / (NCH - kHashFrom);
  static_assert(kPre <= kEarly && kBoundAt > kPre && kDeepAt <= kBoundAt, "lean schedule");
  // the last slot requested before slot s is waited for: kEarly ahead, and
  // every slot of the row from kDeepAt on
  constexpr auto last_issued = [](int s) constexpr {
    if (s < 0) return kEarly - 1;
    const int l = s >= kDeepAt ? NCH - 1 : s + kEarly;
    return l < NCH - 1 ? l : NCH - 1;
  };
  auto issue_slot = [&](int s) {
    const int ch = s * kFT + tid;
    return issue_load_b128(ch < nchunks ? src + ch : &kNegInfChunk);  // lanes past the end load -inf
  };
#pragma unroll
  for (int s = kPre; s < kEarly; ++s) kv[s] = issue_slot(s);
  uint32_t *hash = sh.u32(kLOffHash);
  {  // cleared before the bound's barrier; the histogram and the flag are used after the last slot
    if (hist) {
      uint4 *h4 = (uint4 *)hash;
#pragma unroll
      for (int i = 0; i < kLHashSlots / 4 / kFT; ++i) h4[i * kFT + tid] = make_uint4(0u, 0u, 0u, 0u);
    }
    static_assert(kCandBins == kFT, "one candidate bin per thread");
    sh.u32(kOffCandHist)[tid] = 0u;
    sh.u32(kLOffBinMin)[tid] = 0xFFFFFFFFu;
    if (tid < 2) sh.counters()[kCtrLeanBad + tid] = 0u;
  }
  if (hist) __syncthreads();  // the hash is clear (while the first slots are in flight)
  const uint32_t K = (uint32_t)c.top_k;
  const uint32_t kw = (K + kFW - 1u) / kFW;  // each wave's share of the bound (<= 8)
  bool live = true, tie_below = false;        // (uniform)
  int32_t tv = -0x8000, cmr[kBoundAt], zas = 0x7FFFFFFF;
  uint32_t nacc = 0u, za = 0xFFFFu, y0 = 0u, wrec = 0u;
  uint4 *rec_raw = (uint4 *)sh.u32(kLOffRecRaw) + wave * kRecSeg;
  uint32_t *rec_ch = sh.u32(kLOffRecCh) + wave * kRecSeg;
  auto record = [&](const u32x4 &w, uint32_t ch, bool hit) {  // (all lanes of the wave)
    const uint64_t m = __ballot(hit);
    if (m) {
      const uint32_t pos = wrec + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
      if (hit && pos < (uint32_t)kRecSeg) {
        rec_raw[pos] = make_uint4(w[0], w[1], w[2], w[3]);
        rec_ch[pos] = ch;
      }
      wrec += (uint32_t)__builtin_popcountll(m);
    }
  };
  static_for<0, NCH>([&](auto S) {
    constexpr int s = decltype(S)::value;
    constexpr int last = last_issued(s), prev = last_issued(s - 1);
    static_for<prev + 1, last + 1>([&](auto T) { kv[decltype(T)::value] = issue_slot(decltype(T)::value); });
    // loads issued after slot s's: later slots, and the history ids for the first kPre slots
    constexpr int younger = last - s + (s < kPre ? kHistPer : 0);
    if constexpr (s == kBoundAt) {
      // each wave's kw-th largest running maximum (the largest t with at
      // least kw values >= t, one bit at a time on a uniform t), then the
      // smallest over the waves
      const uint32_t v = (uint32_t)(tv + 0x8000);  // order-preserving in [0, 0xFFFF]
      uint32_t t = 0u;
#pragma unroll
      for (int bit = 15; bit >= 0; --bit) {
        const uint32_t tt = t | (1u << bit);
        if ((uint32_t)__builtin_popcountll(__ballot(v >= tt)) >= kw) t = tt;
      }
      const int32_t lw = (int32_t)t - 0x8000;
      if (lane == 0u) sh.lean_l[wave] = lw;
      __syncthreads();
      int32_t L = sh.lean_l[0];
#pragma unroll
      for (int w = 1; w < kFW; ++w) L = min(L, sh.lean_l[w]);
      L = uniform(L);
      live = L >= 0;  // (a negative bound: the signed maxima do not stand for the values)
      if (live) {
        za = (uint32_t)L | 0x8000u;
        zas = L;
        y0 = temp_key16(za, c);
        // y0's group may hold elements below za, which are not listed
        tie_below = za > 0x8000u && temp_key16(za - 1u, c) == y0;
        // every candidate bin's weight exp(y - y0), while the rest of the row
        // streams in (keys at most 510 apart are at most four binades apart:
        // their f32 difference is exact); a weight that overflows is a
        // reason to decline
        if (tid < kCandBins - 1) {
          const double wt = exp((double)(key16_value(min(y0 + (uint32_t)tid, 0xFFFFu)) - key16_value(y0)));
          ((double *)sh.u32(kLOffWbin))[tid] = wt;
        }
        static_for<0, kBoundAt>([&](auto T) {
          constexpr int t = decltype(T)::value;
          record(kv[t], (uint32_t)(t * kFT + tid), cmr[t] >= zas);
        });
      }
    }
    if constexpr (s >= kHashFrom) {
      // kHashPer history ids a slot into the hash (complete at the barrier
      // after the last slot), before the slot's wait, which hides the
      // atomics' round trips
#pragma unroll
      for (int q = (s - kHashFrom) * kHashPer; q < (s - kHashFrom + 1) * kHashPer && q < kHistPer; ++q)
        if (hist && history_live(q, hid[q], c.h_len, V)) lean_hash_add(hash, hid[q]);
    }
    wait_loads<younger>(kv[s]);
    if constexpr (s == kPre) {  // the history ids were requested before this slot
#pragma unroll
      for (int q = 0; q < kHistPer; ++q) wait_loads<younger>(hid[q]);
    }
    const int32_t cm = chunk_smax(kv[s]);
    nacc = pk_max_u16(nacc, chunk_umax(kv[s]));
    if constexpr (s < kBoundAt) {
      tv = max(tv, cm);
      cmr[s] = cm;
    } else {
      if (live) record(kv[s], (uint32_t)(s * kFT + tid), cm >= zas);
    }
  });
  if (!live) return false;
  // a negative NaN anywhere (positive NaNs are recorded, as they pass za)
  if (max(nacc & 0xFFFFu, nacc >> 16) >= 0xFF81u) atomicOr(&sh.counters()[kCtrLeanBad], 1u);
  // the hash is complete once every wave has passed this barrier
  __syncthreads();
  // every wave lists the candidates of its records
  uint64_t *seg = (uint64_t *)sh.u32(kOffCand) + wave * kCandSeg;
  uint32_t *chist = sh.u32(kOffCandHist);
  uint32_t wn = 0u, ymx = 0u, nan = 0u;
  if (lane < wrec && lane < (uint32_t)kRecSeg) {
    const uint4 raw = rec_raw[lane];
    const uint32_t ch = rec_ch[lane];
    const uint4 kw4 = make_uint4(key_pair(raw.x), key_pair(raw.y), key_pair(raw.z), key_pair(raw.w));
    for (uint32_t e8 = chunk_ge(kw4, za); e8; e8 &= e8 - 1u) {
      const uint32_t e = (uint32_t)__builtin_ctz(e8), idx = ch * 8u + e;
      uint32_t zk = chunk_key(kw4, e);
      if (hist) {
        const uint32_t cnt = lean_hash_count(hash, idx);
        if (cnt) zk = bits_key16(penalise_member(key16_bits(zk), cnt, c));
      }
      nan |= is_nan_key16(zk) ? 1u : 0u;
      // listing positions: every lane in the loop has taken the same
      // iterations, so they all hold the same wn
      const bool put = zk >= za;
      const uint64_t m = __ballot(put);
      if (put) {
        const uint32_t yk = temp_key16(zk, c);
        ymx = max(ymx, yk);
        atomicAdd(&chist[min(yk - y0, (uint32_t)kCandBins - 1u)], 1u);
        atomicMin(&sh.u32(kLOffBinMin)[min(yk - y0, (uint32_t)kCandBins - 1u)], idx);
        const uint32_t pos = wn + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
        if (pos < (uint32_t)kCandSeg) seg[pos] = ((uint64_t)yk << 32) | idx;
      }
      wn += (uint32_t)__builtin_popcountll(m);
    }
  }
  wn = wave_max(wn);
  ymx = wave_max(ymx);
  const bool decline = __ballot(nan != 0u) || wrec > (uint32_t)kRecSeg || wn > (uint32_t)kCandSeg;
  if (lane == 0u) {
    sh.cand_n[wave] = wn;
    // a NaN, or dropped records or candidates: decline
    if (decline) atomicOr(&sh.counters()[kCtrLeanBad], 1u);
    atomicMax(&sh.counters()[kCtrLeanYmax], ymx);
  }
  __syncthreads();
  return stream_finish(sh, a, r, c, K, y0, tie_below);
}

// ---- one row ----------------------------------------------------------------------

// Returns false (uniformly) when the row must go to the generic engine,
// before any output of the row is written.
template <int NCH>
__device__ __forceinline__ bool fast_row(FastShared &sh, const lmrs_sample_args &a, int r) {
  using TR = DTypeTraits<LMRS_DTYPE_BF16>;
  const int tid = threadIdx.x;
  const int64_t V = a.vocab;
  const int nchunks = (int)(V >> 3);
  const int nwords = (int)((V + 31) >> 5);
  const uint32_t npad = (uint32_t)(NCH * kFT - nchunks) * 8u;
  const uint16_t *rowp = (const uint16_t *)((const char *)a.logits + (size_t)r * (size_t)a.row_stride * 2);
  const uint4 *src = (const uint4 *)rowp;
  u32x4 kv[NCH];
  uint32_t k[NCH][4];

  // The row's first kPre slots (their addresses need only the kernel
  // arguments), then the parameters through scalar loads (no store precedes
  // them), the history ids (always kHistPer loads) and the rest of the first
  // kEarly slots.  Requests queue in issue order across the chip: two slots
  // ahead of the parameters hide part of their latency (measured: 0.15 us on
  // C3), eight delay them and the history by more than they gain.  The load
  // pass requests slot s + kEarly when it processes slot s, so that a wave
  // never waits long on a full memory queue with data at hand.  The member
  // tables are built inside the load pass, after slot kHistAt, while the row
  // streams in; the members' raw logits are requested right after them and
  // their keys computed kAhead + 1 slots later.  No path leaves before the
  // load pass consumes the row.
  constexpr int kEarly = NCH / 4;     // slots in flight ahead of the one being processed
  constexpr int kHistAt = 2;          // the slot after which the member tables are built
  constexpr int kAhead = kEarly;      // (a deeper queue from slot kHistAt on measured slower)
  constexpr int kKeysAt = kHistAt + kAhead + 1;  // the slot whose wait covers the members' loads
  constexpr int kPre = 2;             // slots requested before the parameters
  static_assert(kKeysAt < NCH && kAhead >= kEarly && kPre <= kHistAt && kPre <= kEarly,
                "member keys inside the load pass");
  auto issue_slot = [&](int s) {
    const int ch = s * kFT + tid;
    return issue_load_b128(ch < nchunks ? src + ch : &kNegInfChunk);  // lanes past the end load -inf
  };
#pragma unroll
  for (int s = 0; s < kPre; ++s) kv[s] = issue_slot(s);
  const RowCfg c = uniform_cfg(load_row_cfg(a, r, LMRS_DTYPE_BF16));
  // a history longer than the registers hold goes to the generic engine
  // (after the load pass, which every row completes)
  const bool long_hist = c.status == LMRS_ROW_OK && c.hist_on && c.h_len > kFastHistory;
  const bool hist = c.status == LMRS_ROW_OK && c.hist_on && !long_hist;
  uint32_t hid[kHistPer];
  issue_history_ids(hid, a, c, hist, rowp);
  const bool k_on = c.top_k > 0 && c.top_k < V;
  // Greedy and small-k rows whose penalties only lower logits take the lean
  // pass; one that declines is read again by the general pass, in the same
  // order of requests.
  // (not in the widest instantiation: its registers would spill)
  const bool lean = NCH <= 32 && c.status == LMRS_ROW_OK && !long_hist &&
                    (c.greedy || (k_on && c.top_k <= kSmallK)) && penalties_lower(c);
  if constexpr (NCH <= 32) {
    if (lean) {
      if (lean_row<NCH, kPre>(sh, a, r, c, kv, hid, hist, src, nchunks)) return true;
      __syncthreads();  // the lean pass's LDS views are dead
#pragma unroll
      for (int s = 0; s < kPre; ++s) kv[s] = issue_slot(s);
      issue_history_ids(hid, a, c, hist, rowp);
    }
  }
#pragma unroll
  for (int s = kPre; s < kEarly; ++s) kv[s] = issue_slot(s);
  clear_tables(sh, hist, nwords);

  // The load pass: keys, chunk maxima (to LDS as their words fill), the NaN
  // check, and the largest chunk maximum with its slot and keys.
  uint32_t *cml = (uint32_t *)(sh.arena + kOffCm) + tid;
  uint32_t cmw = 0u, mn = 0xFFFFFFFFu, mx = 0u, s1 = 0u, bad = 0u, zmem = 0u, nmem = 0u;
  uint32_t b0 = 0u, b1 = 0u, b2 = 0u, b3 = 0u;  // the keys of chunk s1
  bool mem_ok = false;
  uint32_t mraw[kMemPer];
  static_for<0, NCH>([&](auto S) {
    constexpr int s = decltype(S)::value;
    const int ch = s * kFT + tid;
    // the last slot requested before slot s is waited for
    constexpr int dist = s < kHistAt ? kEarly : kAhead;
    constexpr int last = s + dist < NCH ? s + dist : NCH - 1;
    if constexpr (s < kHistAt) {
      if constexpr (s + kEarly < NCH) kv[s + kEarly] = issue_slot(s + kEarly);
    } else if constexpr (s == kHistAt) {
      static_for<kHistAt + kEarly, last + 1>([&](auto T) { kv[decltype(T)::value] = issue_slot(decltype(T)::value); });
    } else {
      if constexpr (s + kAhead < NCH) kv[s + kAhead] = issue_slot(s + kAhead);
    }
    // loads issued after slot s's: later slots; the history ids for the
    // first kPre slots; the members' for the slots requested before them and
    // waited for after them
    constexpr int younger = last - s + (s > kHistAt && s <= kHistAt + kAhead ? kMemPer : 0) +
                            (s < kPre ? kHistPer : 0);
    wait_loads<younger>(kv[s]);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t kp = key_pair(kv[s][q]);
      k[s][q] = kp;
      mn = pk_min_u16(mn, kp);
    }
    uint32_t cmx = chunk_max(k[s]);
    const bool valid = (s + 1) * kFT <= nchunks || ch < nchunks;
    if (!valid) cmx = 0u;  // padding: no candidates
    const bool top = cmx > mx;  // selects, not branches
    b0 = top ? k[s][0] : b0;
    b1 = top ? k[s][1] : b1;
    b2 = top ? k[s][2] : b2;
    b3 = top ? k[s][3] : b3;
    s1 = top ? (uint32_t)s : s1;
    // made here, while the wave waits for memory anyway (left to itself, the
    // compiler keeps the conditions and selects after the pass)
    asm volatile("" : "+v"(b0), "+v"(b1), "+v"(b2), "+v"(b3), "+v"(s1));
    mx = max(mx, cmx);
    cmw = (s & 1) ? (cmw | (cmx << 16)) : cmx;
    if constexpr ((s & 1) == 1 || s == NCH - 1) cml[(s >> 1) * kFT] = cmw;
    if constexpr (s == kHistAt) {
      // the history ids, followed by slots kPre .. last; waited for on every
      // path (see the member loads below)
      constexpr int hyounger = last - kPre + 1;
#pragma unroll
      for (int q = 0; q < kHistPer; ++q) wait_loads<hyounger>(hid[q]);
      if (hist) {
        mark_history(sh, hid, c.h_len, V);
        nmem = rank_members(sh, nwords);
        if (nmem <= (uint32_t)kFastMembers) count_members(sh, hid, c.h_len, V);
      }
      mem_ok = hist && nmem <= (uint32_t)kFastMembers;
      issue_member_raw(mraw, sh, mem_ok ? nmem : 0u, rowp);  // always kMemPer loads: fixed wait counts
    }
    if constexpr (s == kKeysAt) {
      // Every explicitly issued load is waited for on every path: until its
      // wait, the compiler keeps the destination register for it (a load
      // left unwaited could land in a register already reused).
#pragma unroll
      for (int q = 0; q < kMemPer; ++q) wait_loads<younger>(mraw[q]);
      if (mem_ok) zmem = member_keys(sh, mraw, nmem, c, &bad);
    }
  });
  bad |= mx >= 0xFF81u ? 1u : 0u;
  bad |= min(mn & 0xFFFFu, mn >> 16) <= 0x007Eu ? 1u : 0u;

  if (c.status != LMRS_ROW_OK) {
    if (tid == 0) write_row(a, r, 0u, 0.0f, 0.0f, c.status);
    return true;
  }
  if (long_hist || (hist && !mem_ok)) return false;
  // The thread value: the largest chunk maximum when that chunk holds no
  // member (else none), raised to the members' z keys -- each a distinct
  // element's key.
  const int ft = fresh_tid();
  const uint32_t ch1 = s1 * kFT + (uint32_t)ft;
  const uint32_t tv = max((hist && chunk_m8(sh, ch1) != 0u) ? 0u : mx, zmem);
  uint32_t tvhi = tv, tvlo = tv ? ~tv : 0u;
  block_max3(tvhi, tvlo, bad, sh);
  // Rows with a NaN go to the generic engine: the processors canonicalise
  // NaNs, which the key map does not model.
  if (bad || tvhi == 0u) return false;
  tvlo = ~tvlo;  // the smallest nonzero thread value
  const uint32_t *midx = sh.m_idx(), *mkey = sh.m_key();
  const uint4 *src2 = fresh(src);  // the re-reads
  SelState &ss = sh.ss();

  if (c.greedy || (k_on && c.top_k <= kSmallK)) {  // ---- greedy and small k ----------
    // Greedy (greedy.rs:22-29) is the case k = 1: the first of the sorted candidates.
    const uint32_t K = (uint32_t)c.top_k;
    uint32_t L = tvhi;
    if (K > 1u && !kth_thread(sh, tv, tvhi, tvlo, K, &L)) return false;
    const uint32_t za = group_low(L, c);
    // The chunks whose maximum reaches za give their elements at or above
    // za (members excluded: they enter by their z key) as candidates, as do
    // the members at or above za.  Entry: (~(y key << 16) << 32 | index),
    // whose ascending order is the reference's sorted order.
    uint32_t cw[(NCH + 1) / 2];
#pragma unroll
    for (int w = 0; w < (NCH + 1) / 2; ++w) cw[w] = cm_word(sh, w);  // all reads in flight together
    uint64_t sm = 0u;
    static_for<0, NCH>([&](auto S) {
      constexpr int s = decltype(S)::value;
      sm |= (uint64_t)(((cw[s >> 1] >> (16 * (s & 1))) & 0xFFFFu) >= za ? 1u : 0u) << s;
    });
    uint32_t *ctr = sh.counters();
    auto put = [&](uint32_t zk, uint32_t idx) {
      const uint32_t p = atomicAdd(&ctr[1], 1u);
      if (p < (uint32_t)kGatherCap) ss.gather[p] = ((uint64_t)(~(temp_key16(zk, c) << 16)) << 32) | idx;
    };
    auto chunk_candidates = [&](const uint4 &w, uint32_t ch) {  // w: keys
      for (uint32_t e = chunk_ge(w, za) & ~(hist ? chunk_m8(sh, ch) : 0u); e; e &= e - 1u) {
        const uint32_t el = (uint32_t)__builtin_ctz(e);
        put(chunk_key(w, el), ch * 8u + el);
      }
    };
    // chunk s1 (most often the only one) from the keys the load pass kept;
    // any other from registers, in a pass over the slots that waves without
    // one skip
    if ((sm >> s1) & 1u) chunk_candidates(make_uint4(b0, b1, b2, b3), ch1);
    const uint64_t rest = sm & ~(1ull << s1);
    if (__ballot(rest != 0ull)) {
      static_for<0, NCH>([&](auto S) {
        constexpr int s = decltype(S)::value;
        if ((rest >> s) & 1u) chunk_candidates(make_uint4(k[s][0], k[s][1], k[s][2], k[s][3]), (uint32_t)(s * kFT + ft));
      });
    }
    if (zmem >= za) {  // this thread's members reach za
#pragma unroll
      for (int q = 0; q < kMemPer; ++q) {
        const uint32_t m = (uint32_t)tid + (uint32_t)q * kFT;
        if (m < nmem && (mkey[m] >> 16) >= za) put(mkey[m] >> 16, midx[m]);
      }
    }
    __syncthreads();
    const uint32_t ncand = uniform(ctr[1]);
    if (ncand > (uint32_t)kGatherCap) return false;
    if (ncand <= 64u) {
      // Rank sort: wave w counts, for every candidate i, the candidates
      // 8w .. 8w + 7 smaller than it; wave 0 adds the eight counts and moves
      // candidate i to lane rank(i).
      uint32_t *part = sh.rank_scratch();  // the bitmap is dead
      const uint32_t i = (uint32_t)tid & 63u, j0 = ((uint32_t)tid >> 6) * 8u;
      uint32_t p = 0u;
      if (i < ncand) {
        const uint64_t g = ss.gather[i];
#pragma unroll
        for (uint32_t j = j0; j < j0 + 8u; ++j) p += (j < ncand && ss.gather[j] < g) ? 1u : 0u;
      }
      part[tid] = p;
      __syncthreads();
      if (tid < 64) {
        uint32_t rank = 0u;
#pragma unroll
        for (int w8 = 0; w8 < kFW; ++w8) rank += part[w8 * 64 + tid];
        const uint64_t g = (uint32_t)tid < ncand ? ss.gather[tid] : ~0ull;
        if ((uint32_t)tid >= ncand) rank = (uint32_t)tid;
        const uint32_t lo32 = (uint32_t)__builtin_amdgcn_ds_permute((int)(rank * 4u), (int)(uint32_t)g);
        const uint32_t hi32 = (uint32_t)__builtin_amdgcn_ds_permute((int)(rank * 4u), (int)(uint32_t)(g >> 32));
        finish_wave<TR>(((uint64_t)hi32 << 32) | lo32, c, a, r, K, c.greedy);
      }
      return true;
    }
    if (ncand <= (uint32_t)kFT) {
      // Rank sort: candidate i moves to position (number of smaller
      // candidates) when that is below 64; wave 0 finishes the first K.
      uint64_t *sorted = (uint64_t *)sh.rank_scratch();  // the bitmap is dead
      if ((uint32_t)tid < ncand) {
        const uint64_t g = ss.gather[tid];
        uint32_t rank = 0u;
#pragma unroll 8
        for (uint32_t j = 0; j < ncand; ++j) rank += ss.gather[j] < g ? 1u : 0u;
        if (rank < 64u) sorted[rank] = g;
      }
      __syncthreads();
      if (tid < 64) finish_wave<TR>((uint32_t)tid < ncand ? sorted[tid] : ~0ull, c, a, r, K, c.greedy);
      return true;
    }
    sort_gather<kFT>(ss, ncand);
    finish_sorted<TR, kFT>(ss, c, a, r, K);
    return true;
  }

  // ---- the window of top keys: the full distribution, and top-k cuts whose
  // k-th token lies in it -------------------------------------------------------
  if (full_window<NCH>(sh, a, r, c, k, nchunks, nmem, hist, mx, zmem, tvhi, k_on)) return true;

  if (k_on && c.top_k <= kGatherCap) {  // ---- mid k -------------------------------
    const uint32_t K = (uint32_t)c.top_k;
    uint32_t L;
    if (!kth_value<NCH>(sh, hist, nmem, K, tvhi, &L)) return false;
    const uint32_t za = group_low(L, c);
    // gather every element with z >= za: (~(y key << 16) << 32 | index).
    // Count first (8-bit masks per candidate chunk, packed four to a word),
    // then one scan gives every thread its write offset: no atomics.
    uint32_t masks[(NCH + 3) / 4];
    uint32_t nmine = 0u;
    static_for<0, NCH>([&](auto S) {
      constexpr int s = decltype(S)::value;
      uint32_t m8 = 0u;
      if (((cm_word(sh, s >> 1) >> ((s & 1) * 16)) & 0xFFFFu) >= za) {
#pragma unroll
        for (int e = 0; e < 8; ++e) m8 |= (((k[s][e >> 1] >> ((e & 1) * 16)) & 0xFFFFu) >= za ? 1u : 0u) << e;
        if (hist) m8 &= ~chunk_m8(sh, (uint32_t)(s * kFT + tid));  // members enter by their z key
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
          const uint32_t ch = (uint32_t)(s * kFT + tid);
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
    sort_gather<kFT>(ss, ncand);
    finish_sorted<TR, kFT>(ss, c, a, r, K);
    return true;
  }

  // ---- full: 65536-bin count histogram ------------------------------------------
  __syncthreads();  // the bitmap, chunk maxima and window views are dead
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
#pragma unroll
  for (int s = 0; s < NCH; ++s) {
#pragma unroll
    for (int q = 0; q < 4; ++q) count_word(k[s][q]);
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
  // The entries below overwrite the member list: it waits in registers.
  uint32_t sv_idx[kMemPer], sv_key[kMemPer];
#pragma unroll
  for (int q = 0; q < kMemPer; ++q) {
    const uint32_t m = (uint32_t)tid + (uint32_t)q * kFT;
    sv_idx[q] = m < nmem ? midx[m] : 0u;
    sv_key[q] = m < nmem ? mkey[m] : 0u;
  }
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
  if (c.min_p >= 0.0) {
    // the min-p cut (min_p.rs:45-53): the entries with y at or above the
    // lowest y key it keeps, a prefix of whole tie groups
    const double thr = minp_threshold(M, c);
    if (!(thr == thr)) {  // NaN threshold: softmax_choice of nothing (strategies/mod.rs:28-30)
      if (tid == 0) write_row(a, r, 0u, 0.0f, 0.0f, LMRS_ROW_EMPTY);
      return true;
    }
    const uint32_t ymp = minp_low_key(kNegInfKey16, ykey_of(0), thr, [](uint32_t k) { return key16_value(k); });
    int fm = 0x7FFFFFFF;
    for (int i = E - 1; i >= 0; --i) {
      const int e = tid * E + i;
      if (e < nb && ykey_of(e) < ymp) fm = e;
    }
    fm = block_min<kFW>(fm, sh.iscr);
    if (fm == 0x7FFFFFFF) fm = nb;
    if (fm == 0) {  // not reached: the maximum always passes a non-NaN threshold
      if (tid == 0) write_row(a, r, 0u, 0.0f, 0.0f, LMRS_ROW_EMPTY);
      return true;
    }
    if (fm - 1 < last_h) {  // the cut ends above the top-k set's last tie group
      last_e = fm - 1;
      last_h = group_head(last_e);
      last_keep = cincl[last_e] - cnt_excl(last_h);
      cand_mass = mincl[last_e];
    }
    if (minp_near(key16_value(ymp), M, thr) || (ymp > kNegInfKey16 && minp_near(key16_value(ymp - 1u), M, thr)))
      flags |= LMRS_ROW_NEAR_BOUNDARY;
  }
  // softmax_choice's distribution check (strategies/mod.rs:39-43) on the
  // candidates: a non-finite maximum makes their weights NaN
  if (!(__builtin_isfinite(cand_mass) && cand_mass > 0.0)) {
    if (tid == 0) write_row(a, r, 0u, 0.0f, 0.0f, LMRS_ROW_DISTRIBUTION);
    return true;
  }
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
  const uint32_t kept_n = uniform(cnt_excl(last_h) + last_keep);  // every key is counted here
  __syncthreads();  // entries and prefixes are dead
  if (nmem) {
    uint32_t *wi = sh.m_idx(), *wk = sh.m_key();
#pragma unroll
    for (int q = 0; q < kMemPer; ++q) {
      const uint32_t m = (uint32_t)tid + (uint32_t)q * kFT;
      if (m < nmem) {
        wi[m] = sv_idx[q];
        wk[m] = sv_key[q];
      }
    }
    __syncthreads();
  }
  const uint32_t token = find_jth_stream<NCH>(sh, src2, nchunks, nmem, zlo, zhi, jt);
  if (tid == 0) {
    const double lo_c = (mx2 + (double)(jt - 1u) * wg) / kept_mass, hi_c = lo_c + wg / kept_mass;
    double m = 1.0;
    if (!first_tok && fabs(c.u - lo_c) < m) m = fabs(c.u - lo_c);
    if (!last_tok && fabs(hi_c - c.u) < m) m = fabs(hi_c - c.u);
    if (ovf) m = 0.0;
    write_row(a, r, token, (float)log(wg / kept_mass), yv, flags | (m < 1e-6 ? LMRS_ROW_NEAR_BOUNDARY : 0),
              (int32_t)kept_n, kept_mass);
  }
  return true;
}

__device__ __forceinline__ void launder_args(lmrs_sample_args &a) {
  asm volatile("" : "+s"(a.logits), "+s"(a.dtype), "+s"(a.batch), "+s"(a.vocab), "+s"(a.row_stride));
  asm volatile("" : "+s"(a.hist_offsets), "+s"(a.hist_ids), "+s"(a.repetition_penalty), "+s"(a.presence_penalty));
  asm volatile("" : "+s"(a.frequency_penalty), "+s"(a.temperature), "+s"(a.top_k), "+s"(a.top_p));
  asm volatile("" : "+s"(a.uniforms), "+s"(a.min_p), "+s"(a.token_ids), "+s"(a.log_probs));
  asm volatile("" : "+s"(a.logits_out), "+s"(a.status));
}

// One workgroup per row (the rows in rounds of kRoundWGs, see round_row).
template <int NCH>
__global__ void __launch_bounds__(kFT) bf16_fast_kernel(lmrs_sample_args a) {
  __shared__ FastOrGeneric sh;
  const int r = round_row((int)blockIdx.x, (int)gridDim.x, kRoundWGs);
  if (fast_row<NCH>(sh.f, a, r)) return;
  __syncthreads();
  generic_row<LMRS_DTYPE_BF16, kFT>(sh.g, a, r, 1);
}

// Batches of more rows than CUs (widest rows only): every workgroup takes two
// rows, the rows of slots w and w + G of a grid of G = ceil(n / 2) (round_row:
// the second from the mirrored round, so that an alternating or
// half-and-half batch of cheap and costly rows gives every workgroup one of
// each).  MI355X's in-order dispatch of one workgroup per row left CUs idle
// for up to 46 us between rows while another XCD had no CU free; equal pairs
// keep the CUs of each round finishing together.  The two rows are straight
// code, not a loop: a loop over rows spilled 232 VGPRs, the pair 103
// (C4 176.9 -> 160.7 us).  The arguments pass through an empty asm statement
// before each row, so that nothing derived from them is hoisted across rows
// and held in registers.
template <int NCH>
__device__ __forceinline__ void one_row(FastOrGeneric &sh, const lmrs_sample_args &a0, int r) {
  lmrs_sample_args ar = a0;
  launder_args(ar);
  if (!fast_row<NCH>(sh.f, ar, r)) {
    __syncthreads();
    generic_row<LMRS_DTYPE_BF16, kFT>(sh.g, ar, r, 1);
  }
}

template <int NCH>
__global__ void __launch_bounds__(kFT) bf16_fast_rounds_kernel(lmrs_sample_args a) {
  __shared__ FastOrGeneric sh;
  const int G = (int)gridDim.x;
  const int s0 = (int)blockIdx.x, s1 = s0 + G;
  one_row<NCH>(sh, a, round_row(s0, a.batch, G));
  if (s1 < a.batch) {
    __syncthreads();
    one_row<NCH>(sh, a, round_row(s1, a.batch, G));
  }
}

}  // namespace lmrs
