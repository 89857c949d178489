// lm_head with the sampler in its epilogue (reference: the decode step's
// logits, lm_head(h[:, -1, :]) at transformer/model.py:190 and :201, sampled
// by generation/sampling.py:16-61), for rows that all use top-k.
//
//   prep    one work-group per row: the row's history bitmap (one bit per
//           vocabulary id, which also de-duplicates the ids) and counters;
//   sample  a gemm over every S-th vocabulary row (ns <= 8192 rows,
//           S = ceil(vocab / 8192)), in tiles of 64 rows so that many work-groups
//           share the work; it stores each sampled value's order key.  A
//           logit's value does not depend on its kernel: the same MFMA chain
//           over the same dim order produces it in both gemms;
//   thresh  one work-group per row: the k-th largest sampled key.  The sampled
//           values are a subset of the row's, so at least k of the row's values
//           reach it: a lower bound of the row's k-th largest value;
//   gemm    logits = hidden · weightᵀ on the matrix cores
//           (v_mfma_f32_16x16x32_bf16, fp32 accumulation), one work-group per
//           256 vocabulary rows and every batch row.  The weight streams from
//           HBM once, in whole 128-byte lines, through a double-buffered LDS
//           stage with the hidden states.  Epilogue per logit: bf16
//           rounding (the logits tensor the reference would hold), then
//           soft-cap, penalty and temperature as fl_sample applies them; the
//           values at or above the row's bound are appended to the row's
//           candidates (about k·S of them);
//   pick    one work-group per row: the exact k-th largest candidate by a
//           two-pass radix select, the kept values (ties kept) sorted, then
//           min-p, top-p and the draw with fl_sample's arithmetic.
//
// Traffic: the weight once plus its sampled rows (1/S of it), and the hidden
// states; the [batch, vocab] logits are neither written nor read back.
#include <type_traits>

#include "fl_device.h"
#include "fl_kernels.h"

namespace fl {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int LM_NT = 256;                 // threads of the gemm and pick work-groups
constexpr int LM_NTILE = 256;              // vocabulary rows per gemm tile
constexpr int LM_GW = 8;                   // waves per main-gemm work-group (32 vocabulary rows each)
constexpr int LM_GSLOTS = 2;               // main-gemm stages in flight (register slots)

constexpr int LM_KC = 64;                  // dim per pipeline stage (two MFMA steps of 32)
constexpr int LM_AST = LM_KC + 8;          // LDS row stride of a hidden-state stage, bf16 elements
constexpr int LM_NSAMPLE = 8192;           // sampled vocabulary rows (at most)
constexpr int LM_CAP = FL_LM_HEAD_MAX_CAND;
// Every gemm tile adds its candidate count to each row's counter at the end
// of the kernel; one counter per 256 bytes spreads those atomics over
// channels (64 counters in two cache lines cost ~30 us of serialised atomics
// at 501 tiles x 64 rows).
constexpr int LM_CNT_LD = 64;

// Ascending order key of a 16-bit float pattern: larger value, larger key;
// 0 only for the all-ones NaN pattern (the epilogue maps every NaN to 0).
__device__ __forceinline__ uint32_t asc16(uint32_t bits) { return 0xFFFFu - order16(bits); }
__device__ __forceinline__ uint32_t bits_of_asc16(uint32_t k) { return bits_of_order16(0xFFFFu - k); }
// asc16 keys of -inf and +inf: the non-NaN patterns are exactly the keys
// between them (-NaN patterns lie below, +NaN above)
constexpr uint32_t LM_KEY_NINF = 0x007Fu, LM_KEY_PINF = 0xFF80u;
constexpr uint32_t LM_KEY_NONE = 0x10000u;   // a threshold no key reaches
__device__ __forceinline__ bool bf16_nan(uint32_t bits) { return (bits & 0x7FFFu) > 0x7F80u; }

// A logit's value after soft-cap (cap > 0), the penalty (history members)
// and temperature, as fl_sample evaluates them on a bf16 row, from the
// logit's bf16 pattern.
__device__ __forceinline__ float lm_tval(uint32_t bits, float cap, bool member, float RP, float T, float RT) {
  float z = BF16::to_f32(bits);
  if (cap > 0.0f) z = softcap_val<BF16>(z, cap);
  if (member) z = penalty_val<BF16>(z, RP);
  return temperature_val<BF16>(z, T, RT) + 0.0f;  // (+0.0f: -0 and +0 share a key)
}
__device__ __forceinline__ uint32_t lm_key_of(float y) { return y != y ? 0u : asc16(BF16::from_f32(y)); }

// Smallest key r in [lo, hi] with pred(r) (hi + 1 when none), for pred false
// then true along r; one wave, 64 keys tested per round.
template <class P>
__device__ uint32_t wave_first_key(uint32_t lo, uint32_t hi, P&& pred) {
  const uint32_t lane = threadIdx.x & (WAVE - 1);
  uint32_t end = hi + 1;   // the answer lies in [lo, end]; end: none, or a key known to pass
  while (lo < end) {
    const uint32_t step = (end - lo + WAVE - 1) / WAVE;
    const uint32_t r = lo + step * lane;
    const uint64_t m = __ballot(r < end && pred(r));
    if (m == 0) {
      lo += step * min(static_cast<uint32_t>(WAVE - 1), (end - 1 - lo) / step) + 1;
    } else {
      const uint32_t j = static_cast<uint32_t>(__ffsll(static_cast<unsigned long long>(m)) - 1);
      end = lo + step * j;
      if (j > 0) lo += step * (j - 1) + 1;
    }
  }
  return end;
}

struct LmWs {
  uint32_t* rthr;   // [batch, 4] raw-key thresholds: candidates (non-member, member), +inf (non-member, member)
  uint32_t* cnt;    // [batch, LM_CNT_LD] candidates appended (word 0 of a row's 256 bytes)
  uint32_t* stat;   // [batch] FL_ROW_* bits found by prep and gemm
  uint32_t* bits;   // [batch, bw] history bitmap
  uint16_t* skey;   // [batch, nsl] keys of the sampled rows (entry e: vocabulary row e·S)
  uint64_t* cand;   // [batch, LM_CAP] (key << 32) | ~vocabulary index
  int bw;           // words per bitmap row, a multiple of 4
  int stride;       // S
  int ns;
  int nsl;          // ns rounded up to a multiple of 8
  int prep;         // the call passes a penalty: the prep kernel runs and sets stat
};

__host__ __device__ inline int lm_stride(int64_t vocab) {  // ceil(vocab / 8192): ns <= 8192
  return static_cast<int>((vocab + LM_NSAMPLE - 1) / LM_NSAMPLE);
}
__host__ __device__ inline int lm_ns(int64_t vocab) {
  return static_cast<int>((vocab + lm_stride(vocab) - 1) / lm_stride(vocab));
}
__host__ __device__ inline size_t lm_align(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }
__host__ __device__ inline int lm_bw(int64_t vocab) { return static_cast<int>(((vocab + 31) / 32 + 3) & ~3); }
__host__ __device__ inline int lm_nsl(int64_t vocab) { return (lm_ns(vocab) + 7) & ~7; }
__host__ __device__ inline size_t lm_ws_bytes(int64_t batch, int64_t vocab) {
  const size_t B = static_cast<size_t>(batch), bw = static_cast<size_t>(lm_bw(vocab));
  return lm_align(16 * B) + lm_align(4 * B) + 4 * B * LM_CNT_LD + lm_align(4 * B * bw) +
         lm_align(2 * B * static_cast<size_t>(lm_nsl(vocab))) + 8 * B * LM_CAP;
}
inline LmWs lm_ws(void* p, int64_t batch, int64_t vocab) {
  const size_t B = static_cast<size_t>(batch);
  char* q = static_cast<char*>(p);
  LmWs w;
  w.bw = lm_bw(vocab);
  w.stride = lm_stride(vocab);
  w.ns = lm_ns(vocab);
  w.nsl = lm_nsl(vocab);
  w.prep = 0;
  size_t off = 0;
  w.rthr = reinterpret_cast<uint32_t*>(q + off);
  off += lm_align(16 * B);
  w.cnt = reinterpret_cast<uint32_t*>(q + off);
  off += 4 * B * LM_CNT_LD;
  w.stat = reinterpret_cast<uint32_t*>(q + off);
  off += lm_align(4 * B);
  w.bits = reinterpret_cast<uint32_t*>(q + off);
  off += lm_align(4 * B * w.bw);
  w.skey = reinterpret_cast<uint16_t*>(q + off);
  off += lm_align(2 * B * static_cast<size_t>(w.nsl));
  w.cand = reinterpret_cast<uint64_t*>(q + off);
  return w;
}

__device__ __forceinline__ bool row_penalised(const fl_lm_head_args& a, int b) {
  return a.repetition_penalty != nullptr && a.hist_ids != nullptr && a.hist_len != nullptr &&
         a.repetition_penalty[b] != 1.0f;
}

// Of 256 bin counts, lane holding bins 255 - 4 lane - q in c4[q]: the bin
// where the count from the top reaches k (-1 when the bins hold fewer than k
// keys), and in `above` the count of the bins above it.  Called by a whole wave.
__device__ int wave_top_bin(const uint32_t (&c4)[4], int k, uint32_t& above) {
  const int lane = threadIdx.x & (WAVE - 1);
  const uint32_t s = c4[0] + c4[1] + c4[2] + c4[3];
  const uint32_t incl = wave_incl_scan(s);
  int bin = -1;
  uint32_t run = incl - s;   // keys in higher bins
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (bin < 0 && run + c4[q] >= static_cast<uint32_t>(k)) bin = 255 - 4 * lane - q;
    if (bin < 0) run += c4[q];
  }
  const uint64_t m = __ballot(bin >= 0);
  if (m == 0) return -1;
  const int src = __ffsll(static_cast<unsigned long long>(m)) - 1;
  above = static_cast<uint32_t>(__shfl(static_cast<int>(run), src, WAVE));
  return __shfl(bin, src, WAVE);
}

// The k-th largest of n 16-bit keys (0 when n < k), by one wave: two passes of a 256-bin histogram (high byte, then the
// low byte within the chosen high byte).  hist: 256 words of LDS for this wave.
template <class KeyAt>
__device__ uint32_t wave_kth_key(int n, int k, uint32_t* hist, KeyAt&& key_at) {
  const int lane = threadIdx.x & (WAVE - 1);
  uint32_t prefix = 0;   // high byte, once chosen
  for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
    for (int q = 0; q < 4; ++q) hist[lane + WAVE * q] = 0u;
    __builtin_amdgcn_wave_barrier();
    for (int i = lane; i < n; i += WAVE) {
      const uint32_t key = key_at(i);
      if (pass == 0) atomicAdd(&hist[key >> 8], 1u);
      else if ((key >> 8) == prefix) atomicAdd(&hist[key & 0xFFu], 1u);
    }
    __builtin_amdgcn_wave_barrier();
    uint32_t c4[4], above = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) c4[q] = hist[255 - 4 * lane - q];
    const int bin = wave_top_bin(c4, k, above);
    if (bin < 0) return 0u;   // fewer than k keys
    k -= static_cast<int>(above);
    if (pass == 0) prefix = static_cast<uint32_t>(bin);
    else return (prefix << 8) | static_cast<uint32_t>(bin);
    __builtin_amdgcn_wave_barrier();
  }
  return 0u;
}

}  // namespace

// ---------------------------------------------------------------- prep
// Launched when the call passes a penalty and histories; one work-group per
// row.  A penalised row gets its history bitmap (one bit per vocabulary id,
// which also de-duplicates the ids), built in LDS and written out whole;
// every row gets its status from its history (too long, ids out of range).
__global__ __launch_bounds__(LM_NT) void k_lm_prep(const fl_lm_head_args a, LmWs ws) {
  __shared__ __attribute__((aligned(16))) uint32_t sbits[FL_MAX_VOCAB_16 / 32];   // (bw <= this)
  __shared__ uint32_t s_flags;
  const int b = blockIdx.x, tid = threadIdx.x;
  const bool pen = row_penalised(a, b);
  if (tid == 0) s_flags = 0u;
  int H = pen ? a.hist_len[b] : 0;
  if (pen) {
    uint4* b4 = reinterpret_cast<uint4*>(sbits);
    for (int i = tid; i < ws.bw / 4; i += LM_NT) b4[i] = make_uint4(0u, 0u, 0u, 0u);
  }
  __syncthreads();
  if (H > FL_MAX_HISTORY) {
    if (tid == 0) s_flags = static_cast<uint32_t>(FL_ROW_LIMIT);
    H = 0;
  }
  if (a.hist_ld > 0 && H > a.hist_ld) {  // (a length past its row: the row's ids only)
    if (tid == 0) atomicOr(&s_flags, static_cast<uint32_t>(FL_ROW_BAD_HISTORY));
    H = static_cast<int>(a.hist_ld);
  }
  const int32_t* hid = a.hist_ids + static_cast<int64_t>(b) * a.hist_ld;
  for (int i = tid; i < H; i += LM_NT) {
    const int id = hid[i];
    if (id < 0 || id >= a.vocab) atomicOr(&s_flags, static_cast<uint32_t>(FL_ROW_BAD_HISTORY));
    else atomicOr(&sbits[id >> 5], 1u << (id & 31));
  }
  __syncthreads();
  if (pen) {
    uint4* dst = reinterpret_cast<uint4*>(ws.bits + static_cast<size_t>(b) * ws.bw);
    const uint4* b4 = reinterpret_cast<const uint4*>(sbits);
    for (int i = tid; i < ws.bw / 4; i += LM_NT) dst[i] = b4[i];
  }
  if (tid == 0) ws.stat[b] = s_flags;
}

// ---------------------------------------------------------------- row parameters
// The sample gemm's rows' parameters in LDS, filled once per work-group
// (thread m loads row m's before the gemm's loop, into registers, and stores
// them to LDS after it), so its epilogue computes every key without a memory
// round trip.
template <int MR>
struct LmRows {
  float T[MR], RT[MR], RP[MR];   // temperature, RN(1 / T) (0 for greedy), penalty (1: none)
  uint32_t pen[MR];              // the row is penalised
};
struct LmRowReg {
  float T, RP;
  uint32_t pen;
};
__device__ __forceinline__ LmRowReg lm_row_load(const fl_lm_head_args& a, int m) {
  LmRowReg r{1.0f, 1.0f, 0u};
  if (m < a.batch) {
    r.T = a.temperature[m];
    r.pen = row_penalised(a, m) ? 1u : 0u;
    r.RP = r.pen ? a.repetition_penalty[m] : 1.0f;
  }
  return r;
}
template <int MR>
__device__ __forceinline__ void lm_row_store(LmRows<MR>& p, int m, const LmRowReg& r) {
  p.T[m] = r.T;
  p.RT[m] = r.T > 0.0f ? recip_rt(r.T) : 0.0f;
  p.RP[m] = r.RP;
  p.pen[m] = r.pen;
}

// ---------------------------------------------------------------- sample gemm
// The sampled rows: vocabulary rows e·S for tile entries e, 16 per wave and 64
// per work-group (ns / 64 work-groups), the keys of their transformed values
// stored to ws.skey.  MB: 16-row blocks of the batch (1, 2 or 4).  Each
// 16 x 16 block of logits is one wave's MFMA chain over the dim in 32-wide
// steps in ascending order, as in the main gemm below, so a sampled value
// equals the main gemm's value of the same logit bit for bit.
template <int MB>
__global__ __launch_bounds__(LM_NT) void k_lm_sample(const fl_lm_head_args a, LmWs ws) {
  constexpr int NST = 8;                            // register slots (stages in flight)
  constexpr int MR = 16 * MB;
  constexpr int NE = 16 * (LM_NT / WAVE);          // sampled entries per work-group
  constexpr int BP = MR * NE / LM_NT;              // history words per thread
  __shared__ __attribute__((aligned(16))) uint16_t sA[2][16 * MB * LM_AST];
  __shared__ LmRows<MR> sRows;
  __shared__ uint32_t sBits[MR][NE];                // word of entry j's vocabulary row in row m's bitmap
  const int tid = threadIdx.x, lane = tid & (WAVE - 1), w = tid >> 6;
  const int B = static_cast<int>(a.batch), D = static_cast<int>(a.dim);
  const int S = ws.stride, ns = ws.ns;
  const int e0 = blockIdx.x * NE;
  const int l16 = lane & 15, l4 = lane >> 4;
  const uint16_t* W = static_cast<const uint16_t*>(a.weight);
  // hidden rows 0 .. B-1 (rows of the last block past B read zeros)
  const __amdgpu_buffer_rsrc_t rh =
      row_rsrc(a.hidden, 2u * static_cast<uint32_t>(B - 1) * static_cast<uint32_t>(a.ld_hidden) + 2u * D);

  floatx4 acc[MB][1];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb][0] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  // lane's weight fragment, step ks: tile entry 16 w + l16, vocabulary row
  // (e0 + entry)·S (entries past the end read the last row; their results are
  // dropped), dim k0 + 32 ks + 8 l4 .. +7
  const int eme = e0 + 16 * w + l16;
  const uint16_t* wp = W + static_cast<int64_t>(min(eme, ns - 1)) * S * D + 8 * l4;
  // hidden-state stage: 16 MB rows x 64 columns = 128 MB pieces of 16 bytes
  // (pieces of rows past the batch lie past the buffer's range and read zeros)
  constexpr int GS = LM_KC / 8;
  constexpr int APIECES = (16 * MB * GS + LM_NT - 1) / LM_NT;
  auto load_a = [&](uint4 (&ap)[APIECES], int k0) {
#pragma unroll
    for (int s = 0; s < APIECES; ++s) {
      const int idx = tid + LM_NT * s;
      const int row = idx / GS, seg = idx % GS;
      ap[s] = buf_load16(rh, 2u * (static_cast<uint32_t>(row) * static_cast<uint32_t>(a.ld_hidden) + k0 + 8 * seg), 0u);
    }
  };
  auto store_a = [&](const uint4 (&ap)[APIECES], int st) {
#pragma unroll
    for (int s = 0; s < APIECES; ++s) {
      const int idx = tid + LM_NT * s;
      const int row = idx / GS, seg = idx % GS;
      if (row < 16 * MB) *reinterpret_cast<uint4*>(&sA[st][row * LM_AST + 8 * seg]) = ap[s];
    }
  };
  auto load_w = [&](uint4 (&wf)[2], int k0) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) wf[ks] = *reinterpret_cast<const uint4*>(wp + k0 + 32 * ks);
  };
  auto mfma_stage = [&](int st, const uint4 (&wf)[2]) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const bf16x8 af = *reinterpret_cast<const bf16x8*>(&sA[st][(16 * mb + l16) * LM_AST + 32 * ks + 8 * l4]);
        acc[mb][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, __builtin_bit_cast(bf16x8, wf[ks]), acc[mb][0], 0, 0, 0);
      }
    }
  };

  // the rows' parameters and, for a penalty, the history words of the
  // tile's sampled rows, loaded now and put into LDS after the loop
  const LmRowReg rowp = lm_row_load(a, tid);
  uint32_t bitp[BP];
#pragma unroll
  for (int q = 0; q < BP; ++q) {
    const int i = tid + LM_NT * q, m = i / NE, j = i % NE;
    const int e = min(e0 + j, ns - 1);
    bitp[q] = (ws.prep && m < B) ? ws.bits[static_cast<size_t>(m) * ws.bw + ((e * S) >> 5)] : 0u;
  }

  // Pipeline: stage s (its weight fragments and its hidden pieces) lives in
  // register slot s % NST.  Iteration `it` stores the hidden pieces of stage
  // it + 1 into LDS buffer (it + 1) & 1, multiplies stage it, and refills its
  // slot with stage it + NST, so NST - 1 stages stream from memory during
  // each iteration.  Every load is issued unconditionally, in stage order
  // (past the last stage, the last stage again, never used), and the
  // iterations run in whole groups of NST (those past the last stage only
  // load), so the waits before the LDS stores and the MFMAs leave the later
  // stages in flight.
  const int NIT = D / LM_KC;
  const int NPAD = (NIT + NST - 1) / NST * NST;
  auto kc = [&](int st) { return min(st, NIT - 1) * LM_KC; };
  uint4 wr[NST][2], ar[NST][APIECES];
#pragma unroll
  for (int u = 0; u < NST; ++u) {
    load_w(wr[u], kc(u));
    load_a(ar[u], kc(u));
  }
  store_a(ar[0], 0);
  __syncthreads();
  for (int it0 = 0; it0 < NPAD; it0 += NST) {
#pragma unroll
    for (int u = 0; u < NST; ++u) {
      const int it = it0 + u;
      if (it + 1 < NIT) store_a(ar[(u + 1) % NST], (it + 1) & 1);
      if (it < NIT) mfma_stage(it & 1, wr[u]);
      load_w(wr[u], kc(it + NST));
      load_a(ar[u], kc(it + NST));
      __syncthreads();
    }
  }
  if (tid < MR) lm_row_store(sRows, tid, rowp);
#pragma unroll
  for (int q = 0; q < BP; ++q) {
    const int i = tid + LM_NT * q;
    sBits[i / NE][i % NE] = bitp[q];
  }
  __syncthreads();
  // the sampled values' keys: bf16 rounding (the logit), then soft-cap,
  // penalty and temperature (lm_tval, as the thresholds and the pick apply them)
  const float cap = a.softcap;
  const int n = eme * S;
  uint32_t key[MB][4];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 16 * mb + 4 * l4 + r;
      const bool ok = m < B && eme < ns;
      const bool member = ok && sRows.pen[m] != 0u && ((sBits[m][16 * w + l16] >> (n & 31)) & 1u);
      const float y = lm_tval(BF16::from_f32(acc[mb][0][r]), cap, member, sRows.RP[m], sRows.T[m], sRows.RT[m]);
      key[mb][r] = ok ? lm_key_of(y) : 0u;
    }
  }
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 16 * mb + 4 * l4 + r;
      if (m < B && eme < ns) ws.skey[static_cast<size_t>(m) * ws.nsl + eme] = static_cast<uint16_t>(key[mb][r]);
    }
  }
}

// ---------------------------------------------------------------- main gemm
// logits = hidden · weightᵀ for 256 contiguous vocabulary rows (64 per wave)
// and every batch row, then the epilogue and the candidates at or above each
// row's bound.  A stage is 64 dims of the 256 weight rows and the 16 MB
// hidden rows, staged through LDS twice buffered: each thread loads 16-byte
// pieces (eight lanes cover one 128-byte line of a weight row; the weight
// with the non-temporal policy, read once), stores them to the other buffer
// one iteration later, and the waves read their MFMA fragments from LDS.
// LDS holds 16-byte granule g of row r at r·8 + (g xor ((r >> 1) & 7)): the
// fragment reads (16 rows, one granule column) and the stores (8 granules of
// one row) then spread over all banks.
template <int MB, int NW>
__global__ __launch_bounds__(NW * WAVE) __attribute__((amdgpu_waves_per_eu(NW / 2))) void k_lm_gemm(const fl_lm_head_args a,
                                                                                                   LmWs ws) {
  constexpr int NT = NW * WAVE;
  constexpr int TILE = LM_NTILE;
  constexpr int RW = TILE / NW;                   // weight rows per wave
  constexpr int NB = RW / 16;                     // 16-row weight blocks per wave
  constexpr int MR = 16 * MB;                     // batch rows of the tile
  constexpr int STAGE_Q = (TILE + MR) * 8;        // 16-byte granules per stage
  constexpr int KEYB = MR * TILE * 2;              // epilogue LDS: keys, row parameters, history words
  constexpr int KEY_Q = (KEYB + MR * 16 + MR * 4 + MR * 8 * 4 + 15) / 16;
  static_assert(KEYB % 16 == 0 && MR * 8 <= NT, "epilogue LDS");
  constexpr int SMEM_Q = (2 * STAGE_Q > KEY_Q) ? 2 * STAGE_Q : KEY_Q;
  static_assert(TILE == 16 * NB * NW && LM_KC == 64 && TILE * 8 % NT == 0, "stage shape");
  __shared__ __attribute__((aligned(16))) uint4 smem[SMEM_Q];
  const int tid = threadIdx.x, lane = tid & (WAVE - 1), w = tid >> 6;
  const int B = static_cast<int>(a.batch), D = static_cast<int>(a.dim), V = static_cast<int>(a.vocab);
  const int e0 = blockIdx.x * TILE;
  const int l16 = lane & 15, l4 = lane >> 4;
  const uint16_t* W = static_cast<const uint16_t*>(a.weight);
  const __amdgpu_buffer_rsrc_t rh =
      row_rsrc(a.hidden, 2u * static_cast<uint32_t>(B - 1) * static_cast<uint32_t>(a.ld_hidden) + 2u * D);
  // the tile's weight rows (rows past the vocabulary read zeros)
  const __amdgpu_buffer_rsrc_t rw = row_rsrc(W + static_cast<int64_t>(e0) * D,
                                             2u * static_cast<uint32_t>(min(TILE, V - e0)) * static_cast<uint32_t>(D));
  auto gran = [](int r, int g) { return r * 8 + (g ^ ((r >> 1) & 7)); };

  floatx4 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  // Thread t loads weight rows (t >> 3) + (NT / 8) p, granule t & 7, and
  // hidden pieces t + NT p (row >> 3, granule & 7), into register slot j; the
  // stage's dim k0 goes in the SGPR offset.  Rows past the vocabulary (past
  // the batch) lie past their buffer's range and read zeros: their offset
  // register alone passes the range.
  constexpr int WP = TILE * 8 / NT;
  constexpr int AP = (MR * 8 + NT - 1) / NT;
  uint32_t vw[WP];
#pragma unroll
  for (int p = 0; p < WP; ++p)
    vw[p] = 2u * (static_cast<uint32_t>((tid >> 3) + (NT / 8) * p) * D + 8 * (tid & 7));
  uint32_t va[AP];
#pragma unroll
  for (int p = 0; p < AP; ++p) {
    const int idx = tid + NT * p;
    va[p] = 2u * (static_cast<uint32_t>(idx >> 3) * static_cast<uint32_t>(a.ld_hidden) + 8 * (idx & 7));
  }
  constexpr int NSL = LM_GSLOTS;                   // register slots (stages in flight)
  constexpr int U = NSL % 2 == 0 ? NSL : 2 * NSL;  // iterations per unrolled group
  uint4 wreg[NSL][WP], areg[NSL][AP];
  auto load_stage = [&](int j, int k0) {
#pragma unroll
    for (int p = 0; p < WP; ++p) wreg[j][p] = buf_load16_once(rw, vw[p], 2u * k0);
#pragma unroll
    for (int p = 0; p < AP; ++p) areg[j][p] = buf_load16(rh, va[p], 2u * k0);
  };
  auto store_stage = [&](int j, int st) {
    uint4* sp = smem + st * STAGE_Q;
#pragma unroll
    for (int p = 0; p < WP; ++p) sp[gran((tid >> 3) + (NT / 8) * p, tid & 7)] = wreg[j][p];
#pragma unroll
    for (int p = 0; p < AP; ++p) {
      const int idx = tid + NT * p;
      if ((idx >> 3) < MR) sp[gran(TILE + (idx >> 3), idx & 7)] = areg[j][p];
    }
  };
  auto compute = [&](int st) {
    const uint4* sp = smem + st * STAGE_Q;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8 bfr[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        bfr[nb] = __builtin_bit_cast(bf16x8, sp[gran(RW * w + 16 * nb + l16, 4 * ks + l4)]);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const bf16x8 af = __builtin_bit_cast(bf16x8, sp[gran(TILE + 16 * mb + l16, 4 * ks + l4)]);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bfr[nb], acc[mb][nb], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);   // (one step's fragments live at a time)
    }
  };

  // Pipeline: stage s lives in register slot s % NSL and LDS buffer s & 1.
  // Iteration `it` stores stage it + 1 (loaded NSL iterations earlier) into
  // the buffer the previous iteration read, loads stage it + 1 + NSL into the
  // slot it leaves, then multiplies stage it from LDS: NSL stages stream from
  // HBM during each iteration.  Every load is issued unconditionally, in
  // stage order (past the last stage, the last stage again, never stored),
  // and the iterations run in whole groups of U (those past the last stage
  // only load), so the wait before a store leaves the younger stages in
  // flight.
  // thread m < MR: row m's thresholds and whether it is penalised; thread
  // t < 8 MR: word t & 7 of the tile's 8 history words of row t >> 3 (for a
  // penalty); loaded now, put into LDS after the loop
  constexpr int RPW = MR / NW;   // rows per wave in the candidate append
  static_assert(RPW >= 1 && RPW <= WAVE, "rows per wave");
  uint4 rthr = make_uint4(LM_KEY_NONE, LM_KEY_NONE, LM_KEY_NONE, LM_KEY_NONE);
  uint32_t rpen = 0;
  if (tid < B) {
    rthr = *reinterpret_cast<const uint4*>(ws.rthr + 4 * static_cast<size_t>(tid));
    rpen = row_penalised(a, tid) ? 1u : 0u;
  }
  uint32_t bitw = 0;
  {
    const int m = tid >> 3, wd = (e0 >> 5) + (tid & 7);
    if (ws.prep && tid < 8 * MR && m < B && wd < ws.bw) bitw = ws.bits[static_cast<size_t>(m) * ws.bw + wd];
  }

  const int NIT = D / LM_KC;
  const int NPAD = (NIT + U - 1) / U * U;
  auto kc = [&](int st) { return min(st, NIT - 1) * LM_KC; };
#pragma unroll
  for (int j = 0; j < NSL; ++j) load_stage(j, kc(j));
  store_stage(0, 0);
  load_stage(0, kc(NSL));
  __syncthreads();
  for (int it0 = 0; it0 < NPAD; it0 += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int it = it0 + u;
      if (it + 1 < NIT) store_stage((u + 1) % NSL, (u + 1) & 1);
      load_stage((u + 1) % NSL, kc(it + 1 + NSL));
      if (it < NIT) compute(u & 1);
      __syncthreads();
    }
  }

  // ---------------- epilogue: keys of the tile (LDS reused), then per row the
  // tile's keys at or above the bound appended to the row's candidates
  char* lds = reinterpret_cast<char*>(smem);
  uint16_t (*sKey)[TILE] = reinterpret_cast<uint16_t (*)[TILE]>(lds);
  uint4* sThr = reinterpret_cast<uint4*>(lds + KEYB);
  uint32_t* sPen = reinterpret_cast<uint32_t*>(lds + KEYB + MR * 16);
  uint32_t (*sBits)[8] = reinterpret_cast<uint32_t (*)[8]>(lds + KEYB + MR * 16 + MR * 4);
  if (tid < MR) {
    sThr[tid] = rthr;
    sPen[tid] = rpen;
  }
  if (tid < 8 * MR) sBits[tid >> 3][tid & 7] = bitw;
  __syncthreads();
  // Per value (batch row 16 mb + 4 l4 + r, tile column RW w + 16 nb + l16):
  // its bf16 pattern, whether it is a candidate (the row's threshold for its
  // class reached), and NaN or +inf results for the row's status; then the
  // stores (candidate keys to LDS, the logits, the status bits).
  static_assert(MB * 4 * NB <= 32 && NB % 2 == 0, "epilogue packing");
  uint32_t bits2[MB][4][NB / 2];   // two bf16 patterns per word
  uint32_t cand = 0;               // bit (mb·4 + r)·NB + nb
  uint32_t fnan = 0, finf = 0;     // bit mb·4 + r
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 16 * mb + 4 * l4 + r;
      const bool row_ok = m < B;
      const uint4 th = sThr[m];
      const bool pen = row_ok && sPen[m] != 0u;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int c = RW * w + 16 * nb + l16;
        const bool ok = row_ok && e0 + c < V;
        const uint32_t bits = BF16::from_f32(acc[mb][nb][r]);
        if (nb & 1) bits2[mb][r][nb >> 1] |= bits << 16;
        else bits2[mb][r][nb >> 1] = bits;
        const bool nan = bf16_nan(bits);
        const uint32_t kr = asc16(bits);
        const bool member = pen && ((sBits[m][c >> 5] >> (c & 31)) & 1u);
        const uint32_t tc = member ? th.y : th.x, ti = member ? th.w : th.z;
        const int bit = (mb * 4 + r) * NB + nb;
        cand |= (ok && !nan && kr >= tc) ? (1u << bit) : 0u;
        fnan |= (ok && nan) ? (1u << (mb * 4 + r)) : 0u;
        finf |= (ok && !nan && kr >= ti) ? (1u << (mb * 4 + r)) : 0u;
      }
    }
  }
  uint16_t* out_logits = static_cast<uint16_t*>(a.out_logits);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 16 * mb + 4 * l4 + r;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int c = RW * w + 16 * nb + l16;
        const uint32_t bits = (bits2[mb][r][nb >> 1] >> (16 * (nb & 1))) & 0xFFFFu;
        const bool cd = (cand >> ((mb * 4 + r) * NB + nb)) & 1u;
        sKey[m][c] = static_cast<uint16_t>(cd ? asc16(bits) : 0u);
        if (out_logits != nullptr && m < B && e0 + c < V) out_logits[static_cast<int64_t>(m) * V + e0 + c] = static_cast<uint16_t>(bits);
      }
      const uint32_t f = (((fnan >> (mb * 4 + r)) & 1u) ? static_cast<uint32_t>(FL_ROW_NAN) : 0u) |
                         (((finf >> (mb * 4 + r)) & 1u) ? static_cast<uint32_t>(FL_ROW_INF) : 0u);
      if (f) atomicOr(&ws.stat[m], f);
    }
  }
  __syncthreads();
  // pass 1: per row, the count of the tile's keys at or above its bound
  // (lane i counts row w + NW i); the rows' slots are then claimed by every
  // lane at once
  uint32_t cnt_i = 0;
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int m = w + NW * i;
    if (m >= B) continue;
    int total = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) total += __popcll(__ballot(sKey[m][lane + WAVE * q] != 0u));
    if (lane == i) cnt_i = static_cast<uint32_t>(total);
  }
  uint32_t base_i = 0;
  if (cnt_i > 0) base_i = atomicAdd(&ws.cnt[(w + NW * lane) * LM_CNT_LD], cnt_i);
  // pass 2: the candidates, (raw key << 32) | ~vocabulary index, in tile order
  const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int m = w + NW * i;
    if (!__shfl(static_cast<int>(cnt_i), i, WAVE)) continue;
    uint32_t pos = static_cast<uint32_t>(__shfl(static_cast<int>(base_i), i, WAVE));
    uint64_t* cand = ws.cand + static_cast<size_t>(m) * LM_CAP;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t k = sKey[m][lane + WAVE * q];
      const uint64_t sel = __ballot(k != 0u);
      if ((sel >> lane) & 1ull) {
        const uint32_t p = pos + static_cast<uint32_t>(__popcll(sel & below));
        const uint32_t n = static_cast<uint32_t>(e0 + lane + WAVE * q);
        if (p < static_cast<uint32_t>(LM_CAP)) cand[p] = (static_cast<uint64_t>(k) << 32) | static_cast<uint32_t>(~n);
      }
      pos += static_cast<uint32_t>(__popcll(sel));
    }
  }
}

// ---------------------------------------------------------------- thresh
// The row's bound, then its raw-key thresholds, and the row's counters.
// The bound is the K-th largest of the row's sampled keys (none when fewer
// than K were sampled): the keys go into LDS in 16-byte pieces, then two
// passes of a 256-bin histogram (high byte, then the low byte within the
// chosen high byte), every wave counting into a histogram of its own.
// Soft-cap, penalty and temperature are monotone (non-decreasing) in the
// logit, separately for history members and the rest, so "transformed key
// >= bound" is "raw key >= a threshold" for each class; wave 0 finds the
// thresholds, and those of +inf results (for the row's status), by search
// over the keys of the non-NaN bf16 patterns.  A penalty that is not a
// positive finite number breaks the monotony: such a row reports
// FL_ROW_LIMIT.
__global__ __launch_bounds__(LM_NT) void k_lm_thresh(const fl_lm_head_args a, LmWs ws) {
  constexpr int NW = LM_NT / WAVE;
  __shared__ uint4 keys[LM_NSAMPLE / 8];
  __shared__ uint32_t hist[NW][256];
  __shared__ int s_bin;
  __shared__ uint32_t s_above;
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & (WAVE - 1), w = tid >> 6;
  if (tid == 0) {
    ws.cnt[b * LM_CNT_LD] = 0u;
    if (!ws.prep) ws.stat[b] = 0u;
  }
  const int K = a.top_k[b];
  const bool topk = K >= 1 && K <= FL_LM_HEAD_MAX_TOPK;   // (else the pick reports the row)
  uint32_t bound = 0;   // transformed key; 0: none
  if (topk) {
    const int ns = ws.ns, nq = (ns + 7) >> 3;
    const uint4* src = reinterpret_cast<const uint4*>(ws.skey + static_cast<size_t>(b) * ws.nsl);
    for (int i = tid; i < nq; i += LM_NT) keys[i] = src[i];
    int k = K;
    uint32_t prefix = 0;   // high byte, once chosen
    for (int pass = 0; pass < 2; ++pass) {
      for (int i = tid; i < NW * 256; i += LM_NT) (&hist[0][0])[i] = 0u;
      __syncthreads();   // (pass 0: also the keys)
      for (int i = tid; i < nq; i += LM_NT) {
        const uint4 q = keys[i];
        const uint32_t wd[4] = {q.x, q.y, q.z, q.w};
        const int nj = min(8, ns - 8 * i);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t key = (wd[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
          if (j < nj) {
            if (pass == 0) atomicAdd(&hist[w][key >> 8], 1u);
            else if ((key >> 8) == prefix) atomicAdd(&hist[w][key & 0xFFu], 1u);
          }
        }
      }
      __syncthreads();
      if (w == 0) {
        uint32_t c4[4], above = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          uint32_t c = 0;
#pragma unroll
          for (int v = 0; v < NW; ++v) c += hist[v][255 - 4 * lane - q];
          c4[q] = c;
        }
        const int bin = wave_top_bin(c4, k, above);
        if (lane == 0) {
          s_bin = bin;
          s_above = above;
        }
      }
      __syncthreads();
      const int bin = s_bin;
      if (bin < 0) break;   // fewer than K keys: no bound
      k -= static_cast<int>(s_above);
      if (pass == 0) prefix = static_cast<uint32_t>(bin);
      else bound = (prefix << 8) | static_cast<uint32_t>(bin);
    }
  }
  // wave v finds threshold v: candidates of non-members, of members, +inf
  // of non-members, of members (a row without a penalty has no members)
  static_assert(NW >= 4, "one wave per threshold");
  if (w >= 4) return;
  const float T = a.temperature[b], RT = T > 0.0f ? recip_rt(T) : 0.0f, cap = a.softcap;
  const bool pen = row_penalised(a, b);
  const float RP = pen ? a.repetition_penalty[b] : 1.0f;
  const bool bad = pen && !(RP > 0.0f && RP <= 3.402823466e38f);
  if (w == 0 && bad && lane == 0) atomicOr(&ws.stat[b], static_cast<uint32_t>(FL_ROW_LIMIT));
  const bool member = pen && (w & 1), inf = w >= 2;
  uint32_t t = LM_KEY_NONE;   // (members of a row with a bad penalty: none, the row reports FL_ROW_LIMIT)
  if ((inf || topk) && !(member && bad)) {
    t = wave_first_key(LM_KEY_NINF, LM_KEY_PINF, [&](uint32_t r) {
      const float y = lm_tval(bits_of_asc16(r), cap, member, RP, T, RT);
      return inf ? y == __builtin_inff() : lm_key_of(y) >= bound;
    });
  }
  if (lane == 0) ws.rthr[4 * static_cast<size_t>(b) + w] = t;
}

// ---------------------------------------------------------------- pick
namespace {
// Descending bitonic sort of n (a power of two, 128 .. 1024) 64-bit keys in
// LDS by the work-group.
__device__ void lm_sort_desc(uint64_t* buf, int n) {
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n; i += LM_NT) {
        const int p = i ^ j;
        if (p > i) {
          const uint64_t x = buf[i], y = buf[p];
          const bool desc = (i & k) == 0;
          if (desc ? (x < y) : (x > y)) {
            buf[i] = y;
            buf[p] = x;
          }
        }
      }
      __syncthreads();
    }
  }
}
// The same for 64 keys, one per lane of a wave, through lane shuffles.
__device__ uint64_t wave_sort_desc(uint64_t v) {
  const int lane = threadIdx.x & (WAVE - 1);
  for (int k = 2; k <= WAVE; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      const uint64_t o = shfl_xor(v, j);
      const bool desc = (lane & k) == 0, lower = (lane & j) == 0;
      v = (lower == desc) ? (v > o ? v : o) : (v < o ? v : o);
    }
  }
  return v;
}
constexpr int LM_KEEP = 1024;  // kept values (the k largest and their ties) a row may have
}  // namespace

__global__ __launch_bounds__(LM_NT) void k_lm_pick(const fl_lm_head_args a, LmWs ws) {
  __shared__ uint64_t c[LM_CAP];      // the candidates
  __shared__ uint64_t kept[LM_KEEP];  // the kept ones, sorted
  __shared__ uint32_t sHist[256];
  __shared__ uint32_t s_n, s_nk, s_kth;
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & (WAVE - 1);
  uint32_t status = ws.stat[b];
  const int K = a.top_k[b];
  const uint32_t nc = ws.cnt[b * LM_CNT_LD];
  if (K < 1 || K > FL_LM_HEAD_MAX_TOPK || nc > static_cast<uint32_t>(LM_CAP)) status |= FL_ROW_LIMIT;
  if (tid == 0) {
    s_n = 0;
    s_nk = 0;
  }
  __syncthreads();
  if (status == 0) {
    // each candidate's transformed key (the gemm kept its raw key)
    const float T = a.temperature[b], RT = T > 0.0f ? recip_rt(T) : 0.0f, cap = a.softcap;
    const bool pen = row_penalised(a, b);
    const float RP = pen ? a.repetition_penalty[b] : 1.0f;
    const uint32_t* hb = ws.bits + static_cast<size_t>(b) * ws.bw;
    const uint64_t* cand = ws.cand + static_cast<size_t>(b) * LM_CAP;
    constexpr int G = 4;   // candidates per thread and round: their loads go out together
    for (uint32_t i0 = 0; i0 < nc; i0 += G * LM_NT) {
      uint64_t v[G];
      uint32_t hw[G];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const uint32_t i = i0 + tid + g * LM_NT;
        v[g] = i < nc ? cand[i] : 0ull;
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const uint32_t idx = ~static_cast<uint32_t>(v[g] & 0xFFFFFFFFull);
        hw[g] = (pen && i0 + tid + g * LM_NT < nc) ? hb[idx >> 5] : 0u;
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const uint32_t i = i0 + tid + g * LM_NT;
        if (i < nc) {
          const uint32_t idx = ~static_cast<uint32_t>(v[g] & 0xFFFFFFFFull);
          const bool member = (hw[g] >> (idx & 31)) & 1u;
          const float y = lm_tval(bits_of_asc16(static_cast<uint32_t>(v[g] >> 32)), cap, member, RP, T, RT);
          c[i] = (static_cast<uint64_t>(lm_key_of(y)) << 32) | (v[g] & 0xFFFFFFFFull);
        }
      }
    }
    if (tid == 0) s_n = nc;
  }
  __syncthreads();
  const uint32_t n = s_n;
  if (n > static_cast<uint32_t>(LM_CAP)) status |= FL_ROW_LIMIT;
  // the K-th largest key, then the kept entries (every key at or above it)
  if (status == 0 && tid < WAVE) {
    const uint32_t kth = wave_kth_key(static_cast<int>(n), K, sHist, [&](int i) { return static_cast<uint32_t>(c[i] >> 32); });
    if (lane == 0) s_kth = kth;
  }
  __syncthreads();
  if (status == 0) {
    const uint32_t kth = s_kth;
    for (uint32_t i = tid; i < n; i += LM_NT) {
      if (static_cast<uint32_t>(c[i] >> 32) >= kth) {
        const uint32_t p = atomicAdd(&s_nk, 1u);
        if (p < static_cast<uint32_t>(LM_KEEP)) kept[p] = c[i];
      }
    }
  }
  __syncthreads();
  const int nk_all = static_cast<int>(s_nk);
  if (nk_all > LM_KEEP) status |= FL_ROW_LIMIT;
  const int nk = status == 0 ? nk_all : 0;
  // sorted descending: value, then ascending vocabulary index
  if (nk > WAVE) {
    int np = 128;
    while (np < nk) np <<= 1;
    for (int i = nk + tid; i < np; i += LM_NT) kept[i] = 0ull;
    __syncthreads();
    lm_sort_desc(kept, np);
  } else if (tid < WAVE) {
    const uint64_t v = wave_sort_desc(lane < nk ? kept[lane] : 0ull);
    kept[lane] = v;
  }
  __syncthreads();
  if (tid >= WAVE) return;
  if (status == 0 && nk == 0) status |= FL_ROW_ALL_MASKED;

  // ---------------- decisions (wave 0), fl_sample's arithmetic on the sorted kept values
  const float T = a.temperature[b], TP = a.top_p[b], MP = a.min_p[b];
  const float U = fminf(fmaxf(a.uniforms[b], 0.0f), 0.99999994f);
  auto y_of = [&](int j) { return BF16::to_f32(bits_of_asc16(static_cast<uint32_t>(kept[j] >> 32))); };
  auto idx_of = [&](int j) { return static_cast<int64_t>(~static_cast<uint32_t>(kept[j] & 0xFFFFFFFFull)); };
  const float M = status == 0 ? y_of(0) : 0.0f;
  auto E = [&](int j) { return expf(y_of(j) - M); };
  // fixed-point mass of the first L kept values
  auto mass = [&](int L) {
    uint64_t s = 0;
    for (int j = lane; j < L; j += WAVE) s += to_fx(E(j));
    return wave_reduce(s, OpAdd());
  };
  // first j < L with pred(j) (L if none); pred monotone along j
  auto first = [&](int L, auto&& pred) {
    int f = L;
    for (int j0 = 0; j0 < L && f == L; j0 += WAVE) {
      const uint64_t m = __ballot(j0 + lane < L && pred(j0 + lane));
      if (m) f = j0 + __ffsll(static_cast<unsigned long long>(m)) - 1;
    }
    return f;
  };
  int L = nk;
  int64_t tok = -1;
  float lp = __builtin_nanf("");
  if (status == 0) {
    double S = from_fx(mass(L));
    if (MP > 0.0f) {  // min-p (sampling.py:40-43)
      const float r = 1.0f / static_cast<float>(S);
      const float thr = BF16::rn(BF16::rn(r) * MP);
      const int Lm = first(L, [&](int j) { return BF16::rn(E(j) * r) < thr; });
      if (Lm < L) {
        L = Lm;
        S = from_fx(mass(L));
      }
    }
    if (TP > 0.0f && TP < 1.0f) {  // top-p (sampling.py:45-51)
      const float r1 = 1.0f / static_cast<float>(S);
      const float t = BF16::rn(TP);
      // position j removed when round(round_f32(C_j) - p_j) >= round(top_p),
      // C_j the inclusive cumulative of the rounded probabilities (exact fixed point)
      uint64_t base = 0;
      int cut = L;
      for (int j0 = 0; j0 < L && cut == L; j0 += WAVE) {
        const int j = j0 + lane;
        const float p = j < L ? BF16::rn(E(j) * r1) : 0.0f;
        const uint64_t ci = base + wave_incl_scan(static_cast<uint64_t>(to_fx(p)));
        const bool removed = j < L && BF16::rn(BF16::rn(static_cast<float>(from_fx(ci))) - p) >= t;
        const uint64_t m = __ballot(removed);
        if (m) cut = j0 + __ffsll(static_cast<unsigned long long>(m)) - 1;
        base = readlane64(ci, WAVE - 1);
      }
      L = cut;
    }
    if (L <= 0) {
      status |= FL_ROW_ALL_MASKED;
    } else {
      const double SK = from_fx(mass(L));
      const float rK = 1.0f / static_cast<float>(SK);
      int js = 0;
      if (T <= 0.0f) {
        // greedy (sampling.py:59-60): first index among the maximal rounded probabilities
        const float qmax = BF16::rn(E(0) * rK);
        const int last = first(L, [&](int j) { return BF16::rn(E(j) * rK) != qmax; });
        int64_t best = 0x7fffffffffffffffll;
        for (int j = lane; j < last; j += WAVE) best = min(best, idx_of(j));
        best = wave_reduce(best, OpMin());
        tok = best;
        js = 0;
      } else {
        // inverse CDF over the kept values in descending order (ties by index)
        uint64_t Q = 0;
        for (int j = lane; j < L; j += WAVE) Q += to_fx(BF16::rn(E(j) * rK));
        Q = wave_reduce(Q, OpAdd());
        const uint64_t target = __double2ull_rd(static_cast<double>(U) * static_cast<double>(Q));
        uint64_t base = 0;
        js = -1;
        for (int j0 = 0; j0 < L && js < 0; j0 += WAVE) {
          const int j = j0 + lane;
          const uint64_t q = j < L ? to_fx(BF16::rn(E(j) * rK)) : 0ull;
          const uint64_t ci = base + wave_incl_scan(q);
          const uint64_t m = __ballot(j < L && ci > target);
          if (m) js = j0 + __ffsll(static_cast<unsigned long long>(m)) - 1;
          base = readlane64(ci, WAVE - 1);
        }
        if (js < 0) js = 0;  // (no positive mass: every kept probability rounds to zero)
        tok = idx_of(js);
      }
      // log_softmax(filtered)[tok] as torch evaluates it on a bf16 tensor (sampling.py:97-98)
      const float ysel = T <= 0.0f ? M : y_of(js);
      lp = BF16::rn((ysel - M) - BF16::rn(logf(BF16::rn(static_cast<float>(SK)))));
    }
  }
  if (status != 0) {
    tok = -1;
    lp = __builtin_nanf("");
  }
  if (lane == 0) {
    a.out_token[b] = tok;
    a.out_status[b] = static_cast<int32_t>(status);
    if (a.out_logprob) a.out_logprob[b] = lp;
  }
}

// ---------------------------------------------------------------- launch
size_t lm_head_workspace_bytes(int64_t batch, int64_t vocab) { return lm_ws_bytes(batch, vocab); }

hipError_t launch_lm_head(const fl_lm_head_args& a, hipStream_t s) {
  LmWs ws = lm_ws(a.workspace, a.batch, a.vocab);
  ws.prep = a.repetition_penalty != nullptr && a.hist_ids != nullptr && a.hist_len != nullptr;
  const dim3 rows(static_cast<unsigned>(a.batch));
  if (ws.prep) hipLaunchKernelGGL(k_lm_prep, rows, dim3(LM_NT), 0, s, a, ws);
  const dim3 stiles(static_cast<unsigned>((ws.ns + 63) / 64));
  const dim3 tiles(static_cast<unsigned>((a.vocab + 255) / 256));
  const int mb = static_cast<int>((a.batch + 15) / 16);
  auto run = [&](auto tag_mb) {
    constexpr int MB = decltype(tag_mb)::value;
    hipLaunchKernelGGL((k_lm_sample<MB>), stiles, dim3(LM_NT), 0, s, a, ws);
    hipLaunchKernelGGL(k_lm_thresh, rows, dim3(LM_NT), 0, s, a, ws);
    hipLaunchKernelGGL((k_lm_gemm<MB, LM_GW>), tiles, dim3(LM_GW * WAVE), 0, s, a, ws);
  };
  if (mb <= 1) run(std::integral_constant<int, 1>{});
  else if (mb <= 2) run(std::integral_constant<int, 2>{});
  else run(std::integral_constant<int, 4>{});
  hipLaunchKernelGGL(k_lm_pick, rows, dim3(LM_NT), 0, s, a, ws);
  return hipGetLastError();
}

}  // namespace fl
