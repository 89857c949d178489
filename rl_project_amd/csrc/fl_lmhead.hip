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
#ifndef LM_GW
#define LM_GW 8
#endif
#ifndef LM_GSLOTS
#define LM_GSLOTS 2
#endif
constexpr int LM_KC = 64;                  // dim per pipeline stage (two MFMA steps of 32)
constexpr int LM_AST = LM_KC + 8;          // LDS row stride of a hidden-state stage, bf16 elements
constexpr int LM_NST = 8;                  // weight stages in flight per wave of the sample gemm
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

struct LmWs {
  uint32_t* thr;    // [batch] the row's bound (asc16 key; 0: none)
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
  return 2 * lm_align(4 * B) + 4 * B * LM_CNT_LD + lm_align(4 * B * bw) +
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
  w.thr = reinterpret_cast<uint32_t*>(q + off);
  off += lm_align(4 * B);
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
// which also de-duplicates the ids); every row gets its status from its
// history (too long, ids out of range).
__global__ __launch_bounds__(LM_NT) void k_lm_prep(const fl_lm_head_args a, LmWs ws) {
  __shared__ uint32_t s_flags;
  const int b = blockIdx.x, tid = threadIdx.x;
  uint32_t* bits = ws.bits + static_cast<size_t>(b) * ws.bw;
  const bool pen = row_penalised(a, b);
  if (tid == 0) s_flags = 0u;
  if (pen) {
    uint4* b4 = reinterpret_cast<uint4*>(bits);
    for (int i = tid; i < ws.bw / 4; i += LM_NT) b4[i] = make_uint4(0u, 0u, 0u, 0u);
  }
  __syncthreads();  // (the bitmap's zeros reach memory before the atomics below)
  int H = pen ? a.hist_len[b] : 0;
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
    else atomicOr(&bits[id >> 5], 1u << (id & 31));
  }
  __syncthreads();
  if (tid == 0) ws.stat[b] = s_flags;
}

// ---------------------------------------------------------------- gemm epilogue
// One lane's logits after its MFMA chains: acc[mb][nb][r] is batch row
// 16 mb + 4 l4 + r and vocabulary row col(nb) (negative: past the end).  Each
// value is rounded to bf16 (the logit; stored to out_logits by the main gemm),
// then soft-capped, penalised and divided by the temperature as fl_sample
// does; put(m, nb, key) receives its order key (0 for NaN and out of range).
// The main gemm also records NaN and +inf values in the row's status.
// Two phases: first every key, with loads only (the rows' parameters and
// history bits), then every store.  Global stores among the loads would keep
// the compiler from issuing a later row's loads before an earlier row's
// stores, one memory round trip per row.
template <int MB, int NB, bool SC, bool MAIN, class Col, class Put>
__device__ __forceinline__ void lm_epilogue(const fl_lm_head_args& a, const LmWs& ws, const floatx4 (&acc)[MB][NB],
                                            Col&& col, Put&& put) {
  const int l4 = (threadIdx.x & (WAVE - 1)) >> 4;
  const int B = static_cast<int>(a.batch), V = static_cast<int>(a.vocab);
  const float cap = a.softcap;
  uint32_t key[MB][4][NB], flags[MB][4];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 16 * mb + 4 * l4 + r;
      const bool row_ok = m < B;
      const int mc = row_ok ? m : 0;
      const float T = a.temperature[mc];
      const float RT = T > 0.0f ? 1.0f / T : 0.0f;
      const bool pen = row_ok && row_penalised(a, mc);
      const float RP = pen ? a.repetition_penalty[mc] : 1.0f;
      const uint32_t* hb = ws.bits + static_cast<size_t>(mc) * ws.bw;
      uint32_t f = 0;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int n = col(nb);
        const bool ok = row_ok && n >= 0;
        float z = BF16::to_f32(BF16::from_f32(acc[mb][nb][r]));
        if constexpr (SC) z = softcap_val<BF16>(z, cap);
        if (pen && ok && ((hb[n >> 5] >> (n & 31)) & 1u)) z = penalty_val<BF16>(z, RP);
        const float y = temperature_val<BF16>(z, T, RT) + 0.0f;  // (+0.0f: -0 and +0 share a key)
        const uint32_t yb = BF16::from_f32(y);
        const bool nan = y != y;
        f |= (ok && nan) ? static_cast<uint32_t>(FL_ROW_NAN) : 0u;
        f |= (ok && y == __builtin_inff()) ? static_cast<uint32_t>(FL_ROW_INF) : 0u;
        key[mb][r][nb] = (ok && !nan) ? asc16(yb) : 0u;
      }
      flags[mb][r] = f;
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
        put(m, nb, key[mb][r][nb]);
        const int n = col(nb);
        if (MAIN && out_logits != nullptr && m < B && n >= 0)
          out_logits[static_cast<int64_t>(m) * V + n] = static_cast<uint16_t>(BF16::from_f32(acc[mb][nb][r]));
      }
      if (MAIN && flags[mb][r]) atomicOr(&ws.stat[m], flags[mb][r]);
    }
  }
}

// ---------------------------------------------------------------- sample gemm
// The sampled rows: vocabulary rows e·S for tile entries e, 16 per wave and 64
// per work-group (ns / 64 work-groups), keys stored to ws.skey.  MB: 16-row
// blocks of the batch (1, 2 or 4).  SC: a soft-cap.  Each 16 x 16 block of
// logits is one wave's MFMA chain over the dim in 32-wide steps in ascending
// order, as in the main gemm below, so a sampled value equals the main gemm's
// value of the same logit bit for bit.
template <int MB, bool SC>
__global__ __launch_bounds__(LM_NT) void k_lm_sample(const fl_lm_head_args a, LmWs ws) {
  __shared__ __attribute__((aligned(16))) uint16_t sA[2][16 * MB * LM_AST];
  const int tid = threadIdx.x, lane = tid & (WAVE - 1), w = tid >> 6;
  const int B = static_cast<int>(a.batch), D = static_cast<int>(a.dim);
  const int S = ws.stride, ns = ws.ns;
  const int e0 = blockIdx.x * (LM_NT / WAVE) * 16;
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
  constexpr int APIECES = (16 * MB * LM_KC / 8 + LM_NT - 1) / LM_NT;
  auto load_a = [&](uint4 (&ap)[APIECES], int k0) {
#pragma unroll
    for (int s = 0; s < APIECES; ++s) {
      const int idx = tid + LM_NT * s;
      const int row = idx >> 3, seg = idx & 7;
      ap[s] = buf_load16(rh, 2u * (static_cast<uint32_t>(row) * static_cast<uint32_t>(a.ld_hidden) + k0 + 8 * seg), 0u);
    }
  };
  auto store_a = [&](const uint4 (&ap)[APIECES], int st) {
#pragma unroll
    for (int s = 0; s < APIECES; ++s) {
      const int idx = tid + LM_NT * s;
      const int row = idx >> 3, seg = idx & 7;
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

  // Pipeline: stage s (its weight fragments and its hidden pieces) lives in
  // register slot s % LM_NST.  Iteration `it` stores the hidden pieces of
  // stage it + 1 into LDS buffer (it + 1) & 1, multiplies stage it, and refills
  // its slot with stage it + LM_NST, so LM_NST - 1 stages stream from memory
  // during each iteration.  Every load is issued unconditionally, in stage
  // order (past the last stage, the last stage again, never used), and the
  // iterations run in whole groups of LM_NST (those past the last stage only
  // load), so the waits before the LDS stores and the MFMAs leave the later
  // stages in flight.
  const int NIT = D / LM_KC;
  const int NPAD = (NIT + LM_NST - 1) / LM_NST * LM_NST;
  auto kc = [&](int st) { return min(st, NIT - 1) * LM_KC; };
  uint4 wr[LM_NST][2], ar[LM_NST][APIECES];
#pragma unroll
  for (int u = 0; u < LM_NST; ++u) {
    load_w(wr[u], kc(u));
    load_a(ar[u], kc(u));
  }
  store_a(ar[0], 0);
  __syncthreads();
  for (int it0 = 0; it0 < NPAD; it0 += LM_NST) {
#pragma unroll
    for (int u = 0; u < LM_NST; ++u) {
      const int it = it0 + u;
      if (it + 1 < NIT) store_a(ar[(u + 1) % LM_NST], (it + 1) & 1);
      if (it < NIT) mfma_stage(it & 1, wr[u]);
      load_w(wr[u], kc(it + LM_NST));
      load_a(ar[u], kc(it + LM_NST));
      __syncthreads();
    }
  }
  lm_epilogue<MB, 1, SC, false>(
      a, ws, acc, [&](int) { return eme < ns ? eme * S : -1; },
      [&](int m, int, uint32_t key) {
        if (m < B && eme < ns) ws.skey[static_cast<size_t>(m) * ws.nsl + eme] = static_cast<uint16_t>(key);
      });
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
template <int MB, bool SC, int NW>
__global__ __launch_bounds__(NW * WAVE) __attribute__((amdgpu_waves_per_eu(NW / 2))) void k_lm_gemm(const fl_lm_head_args a,
                                                                                                   LmWs ws) {
  constexpr int NT = NW * WAVE;
  constexpr int TILE = LM_NTILE;
  constexpr int RW = TILE / NW;                   // weight rows per wave
  constexpr int NB = RW / 16;                     // 16-row weight blocks per wave
  constexpr int MR = 16 * MB;                     // batch rows of the tile
  constexpr int STAGE_Q = (TILE + MR) * 8;        // 16-byte granules per stage
  constexpr int KEY_Q = (MR * TILE * 2 + 15) / 16;
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
  // lane i of wave w: row w + NW i's bound, for the candidates after the loop
  constexpr int RPW = MR / NW;
  static_assert(RPW >= 1 && RPW <= WAVE, "rows per wave");
  bool use_i = false;
  uint32_t thr_i = 0;
  if (lane < RPW && w + NW * lane < B) {
    const int K = a.top_k[w + NW * lane];
    use_i = K >= 1 && K <= FL_LM_HEAD_MAX_TOPK;
    thr_i = use_i ? ws.thr[w + NW * lane] : 0u;
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
  uint16_t (*sKey)[TILE] = reinterpret_cast<uint16_t (*)[TILE]>(smem);
  lm_epilogue<MB, NB, SC, true>(
      a, ws, acc,
      [&](int nb) {
        const int n = e0 + RW * w + 16 * nb + l16;
        return n < V ? n : -1;
      },
      [&](int m, int nb, uint32_t key) { sKey[m][RW * w + 16 * nb + l16] = static_cast<uint16_t>(key); });
  __syncthreads();
  // pass 1: per row, the count of the tile's keys at or above its bound
  // (lane i counts row w + NW i); the rows' slots are then claimed by every
  // lane at once
  uint32_t cnt_i = 0;
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int m = w + NW * i;
    const uint32_t thr = static_cast<uint32_t>(__shfl(static_cast<int>(thr_i), i, WAVE));
    if (m >= B || !__shfl(static_cast<int>(use_i), i, WAVE)) continue;
    int total = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t k = sKey[m][lane + WAVE * q];
      total += __popcll(__ballot(k != 0u && k >= thr));
    }
    if (lane == i) cnt_i = static_cast<uint32_t>(total);
  }
  uint32_t base_i = 0;
  if (cnt_i > 0) base_i = atomicAdd(&ws.cnt[(w + NW * lane) * LM_CNT_LD], cnt_i);
  // pass 2: the candidates, (key << 32) | ~vocabulary index, in tile order
  const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int m = w + NW * i;
    if (!__shfl(static_cast<int>(cnt_i), i, WAVE)) continue;
    const uint32_t thr = static_cast<uint32_t>(__shfl(static_cast<int>(thr_i), i, WAVE));
    uint32_t pos = static_cast<uint32_t>(__shfl(static_cast<int>(base_i), i, WAVE));
    uint64_t* cand = ws.cand + static_cast<size_t>(m) * LM_CAP;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t k = sKey[m][lane + WAVE * q];
      const uint64_t sel = __ballot(k != 0u && k >= thr);
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
// The K-th largest of the row's sampled keys (0 when fewer than K were
// sampled), and the row's counters.  The keys go into LDS in 16-byte pieces;
// two passes of a 256-bin histogram follow (high byte, then the low byte
// within the chosen high byte), every wave counting into a histogram of its
// own, and wave 0 finds the bin.
__global__ __launch_bounds__(LM_NT) void k_lm_thresh(const fl_lm_head_args a, LmWs ws) {
  constexpr int NW = LM_NT / WAVE;
  __shared__ uint4 keys[LM_NSAMPLE / 8];
  __shared__ uint32_t hist[NW][256];
  __shared__ int s_bin;
  __shared__ uint32_t s_above;
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & (WAVE - 1), w = tid >> 6;
  if (tid == 0) {
    ws.cnt[b * LM_CNT_LD] = 0u;
    ws.thr[b] = 0u;
    if (!ws.prep) ws.stat[b] = 0u;
  }
  const int K = a.top_k[b];
  if (K < 1 || K > FL_LM_HEAD_MAX_TOPK) return;   // (the pick reports the row)
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
    if (bin < 0) return;   // fewer than K keys: no bound (thr stays 0)
    k -= static_cast<int>(s_above);
    if (pass == 0) {
      prefix = static_cast<uint32_t>(bin);
    } else if (tid == 0) {
      ws.thr[b] = (prefix << 8) | static_cast<uint32_t>(bin);
    }
  }
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
    const uint64_t* cand = ws.cand + static_cast<size_t>(b) * LM_CAP;
    for (uint32_t i = tid; i < nc; i += LM_NT) c[i] = cand[i];
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
  const bool sc = a.softcap > 0.0f;
  const int mb = static_cast<int>((a.batch + 15) / 16);
  auto run = [&](auto tag_mb, auto tag_sc) {
    constexpr int MB = decltype(tag_mb)::value;
    constexpr bool SC = decltype(tag_sc)::value;
    hipLaunchKernelGGL((k_lm_sample<MB, SC>), stiles, dim3(LM_NT), 0, s, a, ws);
    hipLaunchKernelGGL(k_lm_thresh, rows, dim3(LM_NT), 0, s, a, ws);
    hipLaunchKernelGGL((k_lm_gemm<MB, SC, LM_GW>), tiles, dim3(LM_GW * WAVE), 0, s, a, ws);
  };
  using T1 = std::integral_constant<int, 1>;
  using T2 = std::integral_constant<int, 2>;
  using T4 = std::integral_constant<int, 4>;
  if (mb <= 1) sc ? run(T1{}, std::true_type{}) : run(T1{}, std::false_type{});
  else if (mb <= 2) sc ? run(T2{}, std::true_type{}) : run(T2{}, std::false_type{});
  else sc ? run(T4{}, std::true_type{}) : run(T4{}, std::false_type{});
  hipLaunchKernelGGL(k_lm_pick, rows, dim3(LM_NT), 0, s, a, ws);
  return hipGetLastError();
}

}  // namespace fl
