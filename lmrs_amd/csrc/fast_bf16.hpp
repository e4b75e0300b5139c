// fast_bf16.hpp -- the bf16 sampling kernel with the row held in registers.
//
// One workgroup (1024 threads, one per CU at this register and LDS size)
// owns one row of up to NCH * 8192 bf16 logits.  Each thread loads its NCH
// 16-byte chunks (chunk c = s * 1024 + thread) once, in the first few
// microseconds, and converts them in place to 16-bit total-order keys of the
// RAW logits; later passes read registers only.
//
// Penalties never touch the per-element loop.  The history's distinct tokens
// ("members", at most kFastMembers) are found with an LDS hash, their raw
// logits fetched with one scattered load each, and their penalised keys z
// computed in parallel (Repetition then Presence/Frequency, bf16-rounded per
// op, as the reference's chain of kernels).  Every histogram built from the
// raw keys in registers is then corrected by moving each member from its raw
// key to its z key, and every search that matches register keys re-checks
// the (rare) matches against a membership bitmap and adds the members from
// the list.  Temperature is not applied per element either: y = bf16(fma(z,
// 1/T, 0)) is monotone in z, so selection runs on z keys and maps only the
// keys that matter to y (runs of z keys that round to one y form a tie group,
// ordered by index as the reference's sort does).
//
// Paths after the keys are built:
//   greedy   (top_k == 1): lowest index in the maximum's tie group;
//   small k  (top_k <= 4096): a 512-bin histogram of the keys just below the
//            maximum finds the k-th largest key; the candidates (k plus ties)
//            are gathered, sorted exactly and finished in f64;
//   full     (otherwise): a 65536-bin count histogram (two 16-bit counters per
//            LDS word), compacted to its non-empty keys; per-key weights
//            exp(f64(y - max)) times counts give exact cumulative masses for
//            the top-k cut, the nucleus cut and the draw; the chosen token is
//            the j-th lowest index of its tie group, found on a second read
//            of the row.
// Rows this kernel does not take (a NaN anywhere, more than kFastMembers
// distinct history tokens, a histogram count above 65535, more than
// kMaxEntries distinct keys) are marked with token id kDeferred and finished
// by the generic kernel launched right after.
#pragma once

#include "generic_engine.hpp"

namespace lmrs {

constexpr int kWindowBins = 512;
constexpr int kMaxEntries = 6144;   // distinct keys the full path keeps in LDS
constexpr int kFastMembers = 2048;  // distinct history tokens the fast path keeps
constexpr int kFastMaxVocab = 20 * 8192;

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

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
//   [0, 64K)     history hash: token + 1, multiplicity          (history build)
//   [128K, 144K) member list: token ids, raw key | z key << 16  (history build
//                until the full path's compaction; rebuilt for its final search)
//   greedy / small k:  [0, 20K) membership bitmap, [20K, 22K) window histogram,
//                      [24K, 81K) SelState (gather buffer, finish scratch)
//   full:  [0, 128K) 65536 16-bit counters; after compaction [128K, 152K) the
//          entries (key << 16 | count) and [0, 72K) their prefixes; for the
//          final search [0, 20K) bitmap, [20K, 26K) per-slot and per-thread counts
constexpr int kArenaBytes = 152 * 1024;
constexpr int kOffMembers = 128 * 1024;
constexpr int kOffEntries = 128 * 1024;
constexpr int kOffWhist = 20 * 1024;
constexpr int kOffSel = 24 * 1024;
constexpr int kOffSlotCnt = 20 * 1024;
constexpr int kOffTcnt = 22 * 1024;
static_assert(kOffSel + (int)sizeof(SelState) <= kOffMembers, "SelState view");
static_assert(kOffEntries + kMaxEntries * 4 <= kArenaBytes, "entries view");
static_assert(kMaxEntries * 12 <= kOffEntries, "prefix view");

struct FastShared {
  alignas(16) unsigned char arena[kArenaBytes];
  uint32_t chunk_z[8];
  double dscr[kWaves];
  uint32_t uscr[kWaves];
  int32_t iscr[kWaves];
  uint32_t bsel[8];
  RowCfg cfg;

  __device__ uint32_t *u32(int off) { return (uint32_t *)(arena + off); }
  __device__ uint32_t *m_idx() { return u32(kOffMembers); }
  __device__ uint32_t *m_key() { return u32(kOffMembers + kFastMembers * 4); }
  __device__ SelState &ss() { return *(SelState *)(arena + kOffSel); }
};

__device__ __forceinline__ bool member_bit(const uint32_t *bitmap, uint32_t i) {
  return (bitmap[i >> 5] >> (i & 31u)) & 1u;
}

__device__ __forceinline__ void build_bitmap(uint32_t *bitmap, FastShared &sh, uint32_t nmem, int64_t V) {
  const uint32_t *midx = sh.m_idx();
  for (int i = threadIdx.x; i < (int)((V + 31) >> 5); i += kThreads) bitmap[i] = 0u;
  __syncthreads();
  for (uint32_t m = threadIdx.x; m < nmem; m += kThreads) atomicOr(&bitmap[midx[m] >> 5], 1u << (midx[m] & 31u));
  __syncthreads();
}

// Distinct history tokens (< V) of the row with their penalised keys, into
// the member list.  hid holds this thread's history ids (strided by the
// block).  Returns the member count, or kFastMembers + 1 when there are more.
__device__ __forceinline__ uint32_t build_members(FastShared &sh, const uint32_t (&hid)[LMRS_MAX_HISTORY / kThreads],
                                                  const RowCfg &c, int64_t V, const uint16_t *rowp) {
  const int tid = threadIdx.x;
  uint32_t *hkeys = sh.u32(0), *hcnt = sh.u32(kHashCap * 4);
  uint32_t *midx = sh.m_idx(), *mkey = sh.m_key();
  for (int i = tid; i < kHashCap; i += kThreads) {
    hkeys[i] = 0u;
    hcnt[i] = 0u;
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < LMRS_MAX_HISTORY / kThreads; ++q) {
    const uint32_t t = hid[q];
    if ((int64_t)t < V) {
      uint32_t sl = hash_slot(t);
      for (;;) {  // terminates: the table is at most half full
        const uint32_t prev = atomicCAS(&hkeys[sl], 0u, t + 1u);
        if (prev == 0u || prev == t + 1u) {
          atomicAdd(&hcnt[sl], 1u);
          break;
        }
        sl = (sl + 1u) & (kHashCap - 1);
      }
    }
  }
  __syncthreads();
  constexpr int kPer = kHashCap / kThreads;
  uint32_t n = 0, nmem;
#pragma unroll
  for (int i = 0; i < kPer; ++i) n += hkeys[tid * kPer + i] ? 1u : 0u;
  const uint32_t off = block_exclusive_scan(n, sh.uscr, &nmem);
  if (nmem > (uint32_t)kFastMembers) return nmem;
  uint32_t o = off;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const uint32_t key = hkeys[tid * kPer + i];
    if (key) {
      midx[o] = key - 1u;
      mkey[o] = hcnt[tid * kPer + i];  // the count, until replaced below
      ++o;
    }
  }
  __syncthreads();
  // penalised keys, one scattered read of the raw logit per member
  for (uint32_t m = tid; m < nmem; m += kThreads) {
    const uint32_t raw = rowp[midx[m]];
    const uint32_t z = penalise_member(raw, mkey[m], c);
    mkey[m] = bits_key16(raw) | (bits_key16(z) << 16);
  }
  return nmem;
}

// This thread's history ids (strided by the block), 0xFFFFFFFF past the end.
__device__ __forceinline__ void load_history_ids(uint32_t (&hid)[LMRS_MAX_HISTORY / kThreads],
                                                 const lmrs_sample_args &a, const RowCfg &c) {
#pragma unroll
  for (int q = 0; q < LMRS_MAX_HISTORY / kThreads; ++q) {
    const int64_t j = (int64_t)threadIdx.x + (int64_t)q * kThreads;
    hid[q] = j < c.h_len ? a.hist_ids[c.h_begin + j] : 0xFFFFFFFFu;
  }
}

// The j-th (1-based) lowest index among elements whose z key lies in [lo, hi],
// on a second read of the row (raw keys) corrected by the member list.
// Index order is (slot, thread, element): per-slot match counts are reduced
// into LDS, the slot holding the j-th match is found, and one block scan over
// that slot's per-thread counts locates the chunk and then the element.
template <int NCH>
__device__ __forceinline__ uint32_t find_jth_stream(FastShared &sh, const uint4 *src, int nchunks,
                                                    const uint32_t *bitmap, uint32_t nmem,
                                                    uint32_t lo, uint32_t hi, uint32_t j) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t *slot_cnt = sh.u32(kOffSlotCnt), *tcnt = sh.u32(kOffTcnt);
  const uint32_t *midx = sh.m_idx(), *mkey = sh.m_key();
  uint32_t cnt[NCH];
#pragma unroll
  for (int s = 0; s < NCH; ++s) {
    const int ch = s * kThreads + tid;
    cnt[s] = 0u;
    if (ch < nchunks) {
      const uint4 d = src[ch];
      const uint32_t w[4] = {key_pair(d.x), key_pair(d.y), key_pair(d.z), key_pair(d.w)};
      if (chunk_max(w) >= lo) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t key = (w[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
          if (key >= lo && key <= hi && !(nmem && member_bit(bitmap, (uint32_t)(ch * 8 + e)))) cnt[s] += 1u;
        }
      }
    }
  }
  for (int i = tid; i < NCH * kWaves; i += kThreads) slot_cnt[i] = 0u;
  __syncthreads();
#pragma unroll
  for (int s = 0; s < NCH; ++s) {
    const uint32_t t = wave_sum(cnt[s]);
    if (lane == 0 && t) atomicAdd(&slot_cnt[s * kWaves + wave], t);
  }
  for (uint32_t m = tid; m < nmem; m += kThreads) {
    const uint32_t zk = mkey[m] >> 16;
    if (zk >= lo && zk <= hi) {
      const uint32_t ch = midx[m] >> 3;
      atomicAdd(&slot_cnt[(ch >> 10) * kWaves + ((ch & 1023u) >> 6)], 1u);
    }
  }
  __syncthreads();
  if (tid < NCH) {  // per-slot totals
    uint32_t tot = 0;
    for (int w = 0; w < kWaves; ++w) tot += slot_cnt[tid * kWaves + w];
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
  tcnt[tid] = 0u;
  __syncthreads();
  for (uint32_t m = tid; m < nmem; m += kThreads) {  // members of slot sstar, per owner thread
    const uint32_t zk = mkey[m] >> 16;
    const uint32_t ch = midx[m] >> 3;
    if (zk >= lo && zk <= hi && (int)(ch >> 10) == sstar) atomicAdd(&tcnt[ch & 1023u], 1u);
  }
  __syncthreads();
  uint32_t mine = tcnt[tid];
#pragma unroll
  for (int s = 0; s < NCH; ++s)
    if (s == sstar) mine += cnt[s];
  uint32_t tot;
  const uint32_t excl = block_exclusive_scan(mine, sh.uscr, &tot);
  if (excl < jr && jr <= excl + mine) {
    sh.bsel[2] = (uint32_t)(sstar * kThreads + tid);  // the chunk
    sh.bsel[3] = jr - excl;                            // rank inside it
  }
  __syncthreads();
  const uint32_t cstar = uniform(sh.bsel[2]), need0 = uniform(sh.bsel[3]);
  if (tid < 8) sh.chunk_z[tid] = 0xFFFFFFFFu;
  __syncthreads();
  for (uint32_t m = tid; m < nmem; m += kThreads)
    if ((midx[m] >> 3) == cstar) sh.chunk_z[midx[m] & 7u] = mkey[m] >> 16;
  __syncthreads();
  if (tid == 0) {
    const uint4 d = src[cstar];
    const uint32_t w[4] = {key_pair(d.x), key_pair(d.y), key_pair(d.z), key_pair(d.w)};
    uint32_t need = need0, pick = cstar * 8u;
    for (int e = 0; e < 8; ++e) {
      const uint32_t zm = sh.chunk_z[e];
      const uint32_t key = zm != 0xFFFFFFFFu ? zm : ((w[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu);
      if (key >= lo && key <= hi) {
        if (need == 1u) {
          pick = cstar * 8u + (uint32_t)e;
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

template <int NCH>
__global__ void __launch_bounds__(kThreads) bf16_fast_kernel(lmrs_sample_args a) {
  using TR = DTypeTraits<LMRS_DTYPE_BF16>;
  __shared__ FastShared sh;
  const int r = blockIdx.x;
  const int tid = threadIdx.x;
  if (tid == 0) sh.cfg = load_row_cfg(a, r, LMRS_DTYPE_BF16);
  __syncthreads();
  const RowCfg c = uniform_cfg(sh.cfg);
  const int64_t V = a.vocab;
  if (c.status != LMRS_ROW_OK) {
    if (tid == 0) write_row(a, r, 0u, 0.0f, 0.0f, c.status);
    return;
  }
  const int nchunks = (int)(V >> 3);
  const uint32_t npad = (uint32_t)(NCH * kThreads - nchunks) * 8u;
  const uint16_t *rowp = (const uint16_t *)((const char *)a.logits + (size_t)r * (size_t)a.row_stride * 2);
  const uint4 *src = (const uint4 *)rowp;
  const uint32_t *midx = sh.m_idx(), *mkey = sh.m_key();

  // History ids first, so that their loads retire before the logits' loads.
  uint32_t hid[LMRS_MAX_HISTORY / kThreads];
  if (c.hist_on) load_history_ids(hid, a, c);
  uint32_t k[NCH][4];
  // Unconditional loads: lanes past the end re-read the last chunk (no
  // out-of-bounds access, no branches) and are neutralised after conversion.
#pragma unroll
  for (int s = 0; s < NCH; ++s) {
    const uint4 d = src[min(s * kThreads + tid, nchunks - 1)];
    k[s][0] = d.x;
    k[s][1] = d.y;
    k[s][2] = d.z;
    k[s][3] = d.w;
  }
  uint32_t nmem = 0;
  if (c.hist_on) {
    nmem = build_members(sh, hid, c, V, rowp);
    if (nmem > (uint32_t)kFastMembers) {
      if (tid == 0) a.token_ids[r] = kDeferred;
      return;
    }
  }

  // Phase A: raw keys, running max / min (the loads are consumed in order).
  uint32_t mx = 0u, mn = 0xFFFFFFFFu;
#pragma unroll
  for (int s = 0; s < NCH; ++s) {
    const bool valid = (s + 1) * kThreads <= nchunks || s * kThreads + tid < nchunks;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t kp = valid ? key_pair(k[s][q]) : 0u;
      k[s][q] = kp;
      mx = pk_max_u16(mx, kp);
      mn = pk_min_u16(mn, valid ? kp : 0xFFFFFFFFu);
    }
  }
  __syncthreads();  // member keys are complete
  uint32_t mzmax = 0u, mbad = 0u;
  for (uint32_t m = tid; m < nmem; m += kThreads) {
    const uint32_t zk = mkey[m] >> 16;
    mzmax = max(mzmax, zk);
    mbad |= is_nan_key16(zk) ? 1u : 0u;
  }
  const uint32_t rmax = block_max(max(mx & 0xFFFFu, mx >> 16), sh.uscr);
  const uint32_t rmin = block_min(min(mn & 0xFFFFu, mn >> 16), sh.uscr);
  mzmax = block_max(mzmax, sh.uscr);
  mbad = block_max(mbad, sh.uscr);
  // Rows with a NaN go to the generic kernel: the processors canonicalise
  // NaNs, which the key map does not model.
  if (is_nan_key16(rmax) || is_nan_key16(rmin) || mbad) {
    if (tid == 0) a.token_ids[r] = kDeferred;
    return;
  }
  const bool k_on = c.top_k > 0 && c.top_k < V;
  const bool full = !(c.top_k == 1 || (k_on && c.top_k <= kGatherCap));

  if (!full) {
    uint32_t *bitmap = sh.u32(0);
    uint32_t *whist = sh.u32(kOffWhist);
    if (nmem) build_bitmap(bitmap, sh, nmem, V);
    // Window histogram of the 512 keys below the largest z key, from the raw
    // keys in registers corrected by the members.
    const uint32_t hi = max(rmax, mzmax);
    const uint32_t lo = hi >= (uint32_t)(kWindowBins - 1) ? hi - (kWindowBins - 1) : 0u;
    uint32_t zmax = rmax;
    if (nmem || c.top_k != 1) {
      for (int i = tid; i < kWindowBins; i += kThreads) whist[i] = 0u;
      __syncthreads();
#pragma unroll
      for (int s = 0; s < NCH; ++s) {
        if (chunk_max(k[s]) >= lo) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t key = (k[s][e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
            if (key >= lo) atomicAdd(&whist[key - lo], 1u);
          }
        }
      }
      __syncthreads();
      if (tid == 0 && lo == 0u) whist[0] -= npad;  // padding keys
      for (uint32_t m = tid; m < nmem; m += kThreads) {
        const uint32_t rk = mkey[m] & 0xFFFFu, zk = mkey[m] >> 16;
        if (rk >= lo) atomicSub(&whist[rk - lo], 1u);
        if (zk >= lo) atomicAdd(&whist[zk - lo], 1u);
      }
      __syncthreads();
      int top = -1;
      if (tid < kWindowBins && whist[tid]) top = tid;
      top = block_max(top, sh.iscr);
      if (top < 0) {  // every key near the maximum belonged to a penalised member
        if (tid == 0) a.token_ids[r] = kDeferred;
        return;
      }
      zmax = lo + (uint32_t)top;
    }
    const uint32_t ymaxk = temp_key16(zmax, c);
    const float M = key16_value(ymaxk);

    if (c.top_k == 1) {  // ---- greedy (greedy.rs:22-29) -------------------------
      uint32_t za = zmax;
      while (za > 0u && temp_key16(za - 1u, c) == ymaxk) --za;
      uint32_t best = 0xFFFFFFFFu;
#pragma unroll
      for (int s = 0; s < NCH; ++s) {
        const int ch = s * kThreads + tid;
        if (best == 0xFFFFFFFFu && chunk_max(k[s]) >= za) {
#pragma unroll
          for (int e = 7; e >= 0; --e) {
            const uint32_t key = (k[s][e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
            if (key >= za && key <= zmax && !(nmem && member_bit(bitmap, (uint32_t)(ch * 8 + e))))
              best = (uint32_t)(ch * 8 + e);
          }
        }
      }
      for (uint32_t m = tid; m < nmem; m += kThreads) {
        const uint32_t zk = mkey[m] >> 16;
        if (zk >= za && zk <= zmax) best = min(best, midx[m]);
      }
      best = block_min(best, sh.uscr);
      if (tid == 0) write_row(a, r, best, 0.0f, M, LMRS_ROW_OK);
      return;
    }

    // ---- small k: k-th largest z key in the window ----------------------------
    const int d0 = kWindowBins - 1 - 2 * tid, d1 = d0 - 1;
    const uint32_t c0 = d0 >= 0 ? whist[d0] : 0u, c1 = d1 >= 0 ? whist[d1] : 0u;
    uint32_t wtot;
    const uint32_t above0 = block_exclusive_scan(c0 + c1, sh.uscr, &wtot);
    const uint32_t above1 = above0 + c0;
    const uint32_t kk = (uint32_t)c.top_k;
    if (d0 >= 0 && c0 > 0 && above0 < kk && kk <= above0 + c0) sh.bsel[0] = (uint32_t)d0;
    if (d1 >= 0 && c1 > 0 && above1 < kk && kk <= above1 + c1) sh.bsel[0] = (uint32_t)d1;
    __syncthreads();
    if (wtot >= kk) {
      const uint32_t kz = lo + uniform(sh.bsel[0]);
      const uint32_t yk = temp_key16(kz, c);
      uint32_t za = kz;
      while (za > 0u && temp_key16(za - 1u, c) == yk) --za;
      if (za >= lo) {
        // candidates: z keys >= za (the k-th largest's tie group and above)
        const uint32_t ncand =
            block_sum(tid < kWindowBins && (uint32_t)tid >= za - lo ? whist[tid] : 0u, sh.uscr);
        if (ncand <= (uint32_t)kGatherCap) {
          SelState &ss = sh.ss();
          if (tid == 0) sh.bsel[3] = 0u;
          __syncthreads();
#pragma unroll
          for (int s = 0; s < NCH; ++s) {
            if (chunk_max(k[s]) >= za) {
              const int ch = s * kThreads + tid;
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                const uint32_t key = (k[s][e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
                const uint32_t idx = (uint32_t)(ch * 8 + e);
                if (key >= za && !(nmem && member_bit(bitmap, idx))) {
                  const uint32_t slot = atomicAdd(&sh.bsel[3], 1u);
                  ss.gather[slot] = ((uint64_t)(~(temp_key16(key, c) << 16)) << 32) | idx;
                }
              }
            }
          }
          for (uint32_t m = tid; m < nmem; m += kThreads) {
            const uint32_t zk = mkey[m] >> 16;
            if (zk >= za) {
              const uint32_t slot = atomicAdd(&sh.bsel[3], 1u);
              ss.gather[slot] = ((uint64_t)(~(temp_key16(zk, c) << 16)) << 32) | midx[m];
            }
          }
          __syncthreads();
          sort_gather(ss, ncand);
          finish_sorted<TR>(ss, c, a, r, kk);
          return;  // directly: the row's registers are dead on this path
        }
      }
    }
    __syncthreads();
  }

  // ---- full: 65536-bin count histogram --------------------------------------
  uint32_t *h64 = sh.u32(0);
  for (int i = tid; i < 32768; i += kThreads) h64[i] = 0u;
  __syncthreads();
#pragma unroll
  for (int s = 0; s < NCH; ++s) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t w = k[s][q];
      const uint32_t ka = w & 0xFFFFu, kb = w >> 16;
      atomicAdd(&h64[ka & 0x7FFFu], (ka & 0x8000u) ? 0x10000u : 1u);
      atomicAdd(&h64[kb & 0x7FFFu], (kb & 0x8000u) ? 0x10000u : 1u);
    }
  }
  __syncthreads();
  // members move from their raw key to their z key; padding leaves key 0
  for (uint32_t m = tid; m < nmem; m += kThreads) {
    const uint32_t zk = mkey[m] >> 16;
    atomicAdd(&h64[zk & 0x7FFFu], (zk & 0x8000u) ? 0x10000u : 1u);
  }
  __syncthreads();
  for (uint32_t m = tid; m < nmem; m += kThreads) {
    const uint32_t rk = mkey[m] & 0xFFFFu;
    atomicSub(&h64[rk & 0x7FFFu], (rk & 0x8000u) ? 0x10000u : 1u);
  }
  if (tid == 0) atomicSub(&h64[0], npad);
  __syncthreads();
  // Compaction.  Thread t owns the 64 keys 65535-64t .. 65472-64t
  // (descending; position j holds key 65535-64t-j): for t < 512 the high
  // halves of words 32767-64t-j, else the low halves.  Reads are rotated by
  // the thread id so that the 64 lanes of a wave hit 64 different banks.
  const int wbase = 32767 - 64 * (tid & 511);
  const int hsh = tid < 512 ? 16 : 0;
  uint64_t nzmask = 0;
  uint32_t csum = 0;
  for (int jj = 0; jj < 64; ++jj) {
    const int j = (jj + tid) & 63;
    const uint32_t cn = (h64[wbase - j] >> hsh) & 0xFFFFu;
    csum += cn;
    nzmask |= (uint64_t)(cn != 0u) << j;
  }
  uint32_t nbins;
  const uint32_t eoff = block_exclusive_scan((uint32_t)__builtin_popcountll(nzmask), sh.uscr, &nbins);
  const uint32_t total = block_sum(csum, sh.uscr);
  if (total != (uint32_t)V || nbins > (uint32_t)kMaxEntries) {
    // a key with more than 65535 elements, or too many distinct keys
    if (tid == 0) a.token_ids[r] = kDeferred;
    return;
  }
  // entries (key << 16 | count) in descending key order, outside the counters
  uint32_t *ent = sh.u32(kOffEntries);
  for (int jj = 0; jj < 64; ++jj) {
    const int j = (jj + tid) & 63;
    const uint32_t cn = (h64[wbase - j] >> hsh) & 0xFFFFu;
    if (cn) {
      const uint32_t pos = eoff + (uint32_t)__builtin_popcountll(nzmask & ((1ull << j) - 1ull));
      ent[pos] = ((uint32_t)(65535 - 64 * tid - j) << 16) | cn;
    }
  }
  __syncthreads();  // the counters are dead: their space holds the prefixes
  double *mincl = (double *)sh.u32(0);                 // inclusive mass prefix
  uint32_t *cincl = sh.u32(kMaxEntries * 8);           // inclusive count prefix
  const int nb = (int)nbins;
  const int E = (nb + kThreads - 1) / kThreads;  // entries per thread, contiguous
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
  const uint32_t cex = block_exclusive_scan(lc, sh.uscr, &ctot);
  const double mex = block_exclusive_scan(lm, sh.dscr, &mtot);
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
    f = block_min(f, sh.iscr);
    return f == 0x7FFFFFFF ? -1 : f;
  };
  auto first_count = [&](uint32_t target) {
    int f = 0x7FFFFFFF;
    for (int i = E - 1; i >= 0; --i) {
      const int e = tid * E + i;
      if (e < nb && cincl[e] >= target) f = e;
    }
    return block_min(f, sh.iscr);
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
  const uint32_t zhi = ent[h] >> 16, zlo = ent[tl] >> 16;
  const float yv = key16_value(ykey_of(h));
  const bool first_tok = (h == 0 && jt == 1u), last_tok = (h == last_h && jt == gmax);
  __syncthreads();  // entries and prefixes are dead
  uint32_t *bitmap = sh.u32(0);
  if (nmem) {  // the member list was overwritten by the entries: rebuild it
    uint32_t hid2[LMRS_MAX_HISTORY / kThreads];
    load_history_ids(hid2, a, c);
    build_members(sh, hid2, c, V, rowp);
    __syncthreads();
    build_bitmap(bitmap, sh, nmem, V);
  }
  const uint32_t token = find_jth_stream<NCH>(sh, src, nchunks, bitmap, nmem, zlo, zhi, jt);
  if (tid == 0) {
    const double lo_c = (mx2 + (double)(jt - 1u) * wg) / kept_mass, hi_c = lo_c + wg / kept_mass;
    double m = 1.0;
    if (!first_tok && fabs(c.u - lo_c) < m) m = fabs(c.u - lo_c);
    if (!last_tok && fabs(hi_c - c.u) < m) m = fabs(hi_c - c.u);
    if (ovf) m = 0.0;
    write_row(a, r, token, (float)log(wg / kept_mass), yv, flags | (m < 1e-6 ? LMRS_ROW_NEAR_BOUNDARY : 0));
  }
}

}  // namespace lmrs
