// Scaled dot-product self-attention (prefill) for MI355X (gfx950, CDNA4, wave64).
//
// Operator semantics follow the reference contract (contracts/sdpa-1.0.json) and its fp32 reference
// (src/radeon_kernels/ops/sdpa/reference.py:13-38): query, key and value are
// [batch, heads, sequence, head_dim] with one sequence length for all three, query head h reads KV
// head h / (query_heads / kv_heads), scores q.k * scale, an optional causal mask that keeps key j
// for query i when j <= i, fp32 softmax and accumulation, output in the query dtype.  The
// reference itself ships no kernel for this operator (its dispatch is fallback-only,
// dispatch/sdpa-1.0.json); this is a flash-attention forward pass built for CDNA4:
//
//   sdpa_fwd_kernel  one 256-thread workgroup per (sequence, query head, block of 128 queries);
//                    each of its 4 waves owns 32 queries and walks the keys in blocks of BN (64, or
//                    32 for head_dim 256).  K and V
//                    tiles reach LDS by DMA (global_load_lds_dwordx4, no staging registers),
//                    double-buffered: block n + 1 loads while block n is computed, with one
//                    LDS-only barrier per block.  Rows are unpadded and XOR-swizzled in 16-byte
//                    chunks, which keeps both LDS read patterns free of bank conflicts.  Every wave
//                    computes S^T = K Q^T with v_mfma_f32_32x32x16 (K rows from LDS as the A operand,
//                    its queries' Q^T held in registers as the B operand), so each lane owns one
//                    query and 16 keys per 32-key tile and the softmax needs one exchange between
//                    the two wave halves; the probabilities, rounded to the input dtype, are already
//                    laid out as the B operand of O^T += V^T P^T, whose A operand comes from
//                    ds_read_b64_tr_b16 transposing reads of the row-major V tile (the keys of one
//                    MFMA k-step are taken in the order the S^T accumulator holds them, which the
//                    transposing read reproduces by the addresses it is given).  Masking runs only
//                    on blocks that hold a masked key.  The softmax reference may lag the running
//                    maximum by a bounded slack, so the accumulator is rescaled only when some
//                    query's maximum outgrows it -- in practice in the first blocks.  With the
//                    causal mask, blocks past a wave's last query are skipped and the grid runs the
//                    longest query blocks of every head first (1.7x over head-major order on the long
//                    causal case); without it, neighbouring query blocks of one head run together
//                    and share its K and V rows in L2.
//
// Scores are kept in the base-2 domain: p = exp2((q . k) * scale * log2(e) - m), evaluated as one
// fused multiply-add per score; the block maximum is taken on the raw dot products (scale > 0 keeps
// their order) and scaled once per block.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <numeric>
#include <string>
#include <utility>

#include "rk_sdpa.h"

namespace {

constexpr int kWave = 64;
constexpr int kWaves = 4;
constexpr int kThreads = kWave * kWaves;
constexpr int kBlockM = 128;  // queries per workgroup (32 per wave)
constexpr float kLog2e = 1.4426950408889634f;
// How far (log2 units) the softmax reference may trail the running maximum before a rescale.
constexpr float kRescaleSlack = 8.0f;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

struct Bf16 {
  // Round to nearest even, both halves in one v_cvt_pk_bf16_f32.
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
  }
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   c, 0, 0, 0);
  }
};

struct Fp16 {
  // Round to nearest even, both halves in one v_cvt_pk_f16_f32.
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, f16x2));
  }
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  }
};

__device__ __forceinline__ uint32_t bits(float x) { return __builtin_bit_cast(uint32_t, x); }
// v_exp_f32: 2^x (exp2(-inf) = 0).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fbits(uint32_t x) { return __builtin_bit_cast(float, x); }

// v_permlane32_swap with the same value in both operands yields {x[l & ~32], x[l | 32]}: combining
// the pair gives the reduction over the two wave halves, identical in both.
__device__ __forceinline__ float max_halves(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(bits(x), bits(x), false, false);
  return fmaxf(fbits(r[0]), fbits(r[1]));
}
__device__ __forceinline__ float sum_halves(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(bits(x), bits(x), false, false);
  return fbits(r[0]) + fbits(r[1]);
}

struct Params {
  const uint16_t* __restrict__ q;  // [B, Hq, S, D]
  const uint16_t* __restrict__ k;  // [B, Hkv, S, D]
  const uint16_t* __restrict__ v;  // [B, Hkv, S, D]
  uint16_t* __restrict__ out;      // [B, Hq, S, D]
  int32_t batch, query_heads, kv_heads, group, seq, q_blocks;
  int32_t xcd_slices;   // 0: two-dimensional grid; else 1-D grid, every XCD owning whole group slices
  int32_t slice_items;  // workgroups of one group slice: group * ceil(q_blocks / xcd_slices)
  float scale_log2e;
};

// s_waitcnt immediates (gfx9 encoding: vmcnt in bits [3:0] and [15:14], expcnt [6:4], lgkmcnt
// [11:8]): all vector memory operations done, and all LDS operations done.
constexpr int kWaitVmcnt0 = 0x0F70;
constexpr int kWaitLgkmcnt0 = 0xC07F;

// Keys per block BN and workgroups per CU.  head_dim 256 takes 32-key blocks (its four tiles then stay
// within the 64 KB the ds offset field addresses) at one workgroup per CU, whose 512 registers per
// lane hold its accumulators without spilling (two per CU spilled and ran 5-9% slower).  head_dim
// 64 and 128 take 64-key blocks at two workgroups per CU (fewer barriers per key).  A 32-key form of
// head_dim 128 at three workgroups per CU was faster on grids of several rounds only while those
// grids re-streamed K/V past L2; with the XCD-owned grid order the 64-key form is 0.3-3% faster
// there too, so it is the only one built.
template <int D, int BN>
struct Tiling {
  static_assert(BN == 32 || BN == 64, "32 or 64 keys per block");
  static_assert(D != 256 || BN == 32, "head_dim 256 uses 32-key blocks");
  static constexpr int kBlockN = BN;
  static constexpr int kOccupancy = D == 256 ? 1 : 2;  // resident workgroups per CU
  static constexpr int kRowBytes = D * 2;
  static constexpr int kTileBytes = kBlockN * kRowBytes;  // one K or V tile
  static constexpr int kDmaPerWave = kTileBytes / 1024 / kWaves;  // 1 KB per DMA instruction
  static_assert(kDmaPerWave * 1024 * kWaves == kTileBytes, "tile must split into whole DMA instructions");
};

// LDS placement: 16-byte chunk c of tile row r sits in slot c ^ swizzle(r) of that row.  The
// swizzle makes both LDS read patterns bank-conflict free: the K operand reads (16 consecutive rows,
// one chunk) see 16 distinct slots (distinct bank groups once rows of 128 bytes pair up), and the
// transposing V reads (4 consecutive rows, 4 consecutive chunks) see 16 distinct slots because the
// swizzle of 4 consecutive rows differs in bits 2-3 (in bit 2 within each row parity for head_dim
// 64, whose two rows share one 256-byte bank line).
template <int D>
__device__ __forceinline__ int swizzle(int r) {
  if constexpr (D == 64)
    return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
  else
    return ((r & 3) << 2) | ((r >> 2) & 3);
}

// global_load_lds_dwordx4: each lane's 16 bytes at `src` land in LDS at `lds_base` + 16 * lane
// (`lds_base` wave-uniform); completion is tracked by the wave's vector memory counter.
__device__ __forceinline__ void dma16(const void* src, void* lds_base) {
  __builtin_amdgcn_global_load_lds(src, lds_base, 16, 0, 0);
}

// Workgroup barrier that orders LDS accesses but leaves outstanding global loads (the next
// block's DMA) in flight, unlike __syncthreads.
__device__ __forceinline__ void lds_barrier() {
  __asm__ __volatile__("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(kWaitLgkmcnt0);
  __builtin_amdgcn_s_barrier();
  __asm__ __volatile__("" ::: "memory");
}

__device__ __forceinline__ uint32_t lds_address(const void* ptr) {
  typedef const __attribute__((address_space(3))) char lds_char;
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_char*)(ptr)));
}

// LDS reads issued as inline assembly with their own lgkmcnt wait.  The compiler places a vmcnt(0)
// wait in front of every LDS read it emits while an LDS DMA is outstanding (it cannot tell which
// bytes the DMA writes), which would stall on the next block's tiles; these reads only ever touch
// the current block's buffer, whose DMA an explicit wait has already covered.  OFFSET (the buffer
// and tile position, a compile-time constant) goes into the instruction's immediate offset field,
// so each lane keeps only its swizzled per-k-step offsets in registers.
template <int OFFSET>
__device__ __forceinline__ void lds_read_b128_x4(u32x4 (&a)[4], const uint32_t* addr) {
  static_assert(OFFSET >= 0 && OFFSET < 65536, "ds offset field");
  __asm__ __volatile__(
      "ds_read_b128 %0, %4 offset:%8\n\t"
      "ds_read_b128 %1, %5 offset:%8\n\t"
      "ds_read_b128 %2, %6 offset:%8\n\t"
      "ds_read_b128 %3, %7 offset:%8\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(a[0]), "=&v"(a[1]), "=&v"(a[2]), "=&v"(a[3])
      : "v"(addr[0]), "v"(addr[1]), "v"(addr[2]), "v"(addr[3]), "i"(OFFSET)
      : "memory");
}

// Transposing 64-bit reads for two 32-dim tiles of one 16-key k-step: rows r and r + 8 of each
// tile form one MFMA A operand.
template <int OFFSET>
__device__ __forceinline__ void lds_read_tr_x2(u32x4 (&a)[2], const uint32_t* lo, const uint32_t* hi) {
  static_assert(OFFSET >= 0 && OFFSET < 65536, "ds offset field");
  u32x2 r[4];
  __asm__ __volatile__(
      "ds_read_b64_tr_b16 %0, %4 offset:%8\n\t"
      "ds_read_b64_tr_b16 %1, %5 offset:%8\n\t"
      "ds_read_b64_tr_b16 %2, %6 offset:%8\n\t"
      "ds_read_b64_tr_b16 %3, %7 offset:%8\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
      : "v"(lo[0]), "v"(hi[0]), "v"(lo[1]), "v"(hi[1]), "i"(OFFSET)
      : "memory");
  a[0] = u32x4{r[0][0], r[0][1], r[1][0], r[1][1]};
  a[1] = u32x4{r[2][0], r[2][1], r[3][0], r[3][1]};
}

template <int OFFSET>
__device__ __forceinline__ void lds_read_tr_x4(u32x4 (&a)[4], const uint32_t* lo, const uint32_t* hi) {
  static_assert(OFFSET >= 0 && OFFSET < 65536, "ds offset field");
  u32x2 r[8];
  __asm__ __volatile__(
      "ds_read_b64_tr_b16 %0, %8 offset:%16\n\t"
      "ds_read_b64_tr_b16 %1, %9 offset:%16\n\t"
      "ds_read_b64_tr_b16 %2, %10 offset:%16\n\t"
      "ds_read_b64_tr_b16 %3, %11 offset:%16\n\t"
      "ds_read_b64_tr_b16 %4, %12 offset:%16\n\t"
      "ds_read_b64_tr_b16 %5, %13 offset:%16\n\t"
      "ds_read_b64_tr_b16 %6, %14 offset:%16\n\t"
      "ds_read_b64_tr_b16 %7, %15 offset:%16\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7])
      : "v"(lo[0]), "v"(hi[0]), "v"(lo[1]), "v"(hi[1]), "v"(lo[2]), "v"(hi[2]), "v"(lo[3]), "v"(hi[3]),
        "i"(OFFSET)
      : "memory");
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = u32x4{r[2 * i][0], r[2 * i][1], r[2 * i + 1][0], r[2 * i + 1][1]};
}

template <int N>
struct Int {
  static constexpr int value = N;
};

// f(Int<0>{}), ..., f(Int<N - 1>{}): loop indices usable as constant expressions.
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(Int<I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

template <class E, int D, int BLOCK_N, bool CAUSAL>
__global__ __launch_bounds__(kThreads, (Tiling<D, BLOCK_N>::kOccupancy)) void sdpa_fwd_kernel(Params p) {
  static_assert(D == 64 || D == 128 || D == 256, "head_dim must be 64, 128 or 256");
  using T = Tiling<D, BLOCK_N>;
  constexpr int BN = T::kBlockN;
  constexpr int KS = D / 16;    // MFMA k-steps of S^T (16 dims each)
  constexpr int DT = D / 32;    // 32-dim tiles of O^T
  constexpr int ST = BN / 32;   // 32-key tiles of S^T per block
  constexpr int PK = BN / 16;   // 16-key k-steps of O^T += V^T P^T per block
  constexpr int RB = T::kRowBytes;
  constexpr int TB = T::kTileBytes;
  constexpr int NDMA = T::kDmaPerWave;
  // Double-buffered K and V tiles, filled by DMA: the next block's loads run under this block's
  // math.  Buffer u holds K at byte 2 u TB and V at (2 u + 1) TB.
  __shared__ __attribute__((aligned(1024))) unsigned char lds[4 * TB];
  static_assert(4 * TB <= 65536, "buffer offsets must fit the ds offset field");

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int col = lane & 31;

  // Grid -> (sequence, query head, query block).
  //   xcd_slices = S > 0 (grids of several rounds): a KV group (sequence x KV head) is cut into S
  //     slices by query-block residue (S = 8 / gcd(groups, 8), 1 when the groups divide into 8), so
  //     the slices divide into 8.  The dispatcher places hardware workgroup h on XCD h % 8, so XCD x
  //     takes slices x, x + 8, ... one after the other; within a slice the query blocks go in order
  //     (causal: longest first, the key range grows with the query block), the group's query heads
  //     adjacent.  The workgroups resident on one XCD then read one or two groups' K/V (2 MB each at
  //     S = 4096, D = 128) out of its 4 MB L2.  In the two-dimensional orders below every XCD holds
  //     blocks of all groups at once and re-streams K/V past its L2: 2.9 GB of L2 fetches per call
  //     on the 4-sequence, 32x8-head, S = 4096 causal case, for 201 MB of Q, K and V.  Slices hold
  //     ceil(q_blocks / S) blocks; the padding workgroups of shorter slices exit at once.
  //   Otherwise, causal: x = (sequence, head), y = query block, longest first; noncausal:
  //     x = query block, y = (sequence, head).
  int bh, qb;
  if (p.xcd_slices > 0) {
    const int hw = static_cast<int>(blockIdx.x);
    const int local = (hw >> 3) / p.slice_items;   // the XCD's local-th slice
    const int r = (hw >> 3) - local * p.slice_items;
    const int vslice = local * 8 + (hw & 7);
    const int kv_group = vslice / p.xcd_slices;    // b * Hkv + hkv
    const int residue = vslice - kv_group * p.xcd_slices;
    const int rank = r / p.group;
    const int ordinal = rank * p.xcd_slices + residue;  // position in the group's block order
    if (ordinal >= p.q_blocks) return;                   // padding
    qb = CAUSAL ? p.q_blocks - 1 - ordinal : ordinal;
    const int seq_index = kv_group / p.kv_heads;
    bh = seq_index * p.query_heads + (kv_group - seq_index * p.kv_heads) * p.group + (r - rank * p.group);
  } else {
    bh = CAUSAL ? static_cast<int>(blockIdx.x) : static_cast<int>(blockIdx.y);  // b * Hq + hq
    qb = CAUSAL ? p.q_blocks - 1 - static_cast<int>(blockIdx.y) : static_cast<int>(blockIdx.x);
  }
  const int b = bh / p.query_heads;
  const int hq = bh - b * p.query_heads;
  const int hkv = hq / p.group;
  const int S = p.seq;
  const int q_wave = qb * kBlockM + wave * 32;  // first query of this wave
  const int my_q = q_wave + col;                // the query this lane owns

  const uint16_t* __restrict__ qrow = p.q + (static_cast<int64_t>(bh) * S + min(my_q, S - 1)) * D;
  const uint16_t* __restrict__ kbase_ptr = p.k + static_cast<int64_t>(b * p.kv_heads + hkv) * S * D;
  const uint16_t* __restrict__ vbase_ptr = p.v + static_cast<int64_t>(b * p.kv_heads + hkv) * S * D;

  const int kv_end = CAUSAL ? min(S, (qb + 1) * kBlockM) : S;
  const int n_blocks = (kv_end + BN - 1) / BN;

  // DMA sources: instruction i of this wave fills tile bytes [(wave * NDMA + i) KB, +1 KB); lane L
  // lands at byte 16 L of it, i.e. row r, slot s, and fetches the row's chunk s ^ swizzle(r).
  int dma_row[NDMA], dma_col[NDMA];
#pragma unroll
  for (int i = 0; i < NDMA; ++i) {
    const int offset = (wave * NDMA + i) * 1024 + 16 * lane;
    const int r = offset / RB, slot = (offset % RB) / 16;
    dma_row[i] = r;
    dma_col[i] = (slot ^ swizzle<D>(r)) * 8;
  }
  auto issue = [&](int kb0, int buffer) {
    unsigned char* k_tile = lds + 2 * buffer * TB;
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      // Rows past the sequence re-read its last row (in bounds); their scores are masked and their
      // V rows zeroed before use.
      const int64_t offset = static_cast<int64_t>(min(kb0 + dma_row[i], S - 1)) * D + dma_col[i];
      dma16(kbase_ptr + offset, k_tile + (wave * NDMA + i) * 1024);
      dma16(vbase_ptr + offset, k_tile + TB + (wave * NDMA + i) * 1024);
    }
  };
  issue(0, 0);  // in flight while Q is loaded

  // B operand of S^T = K Q^T: column = this lane's query, k-chunk (half) of 8 dims per k-step.
  u32x4 qB[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const u32x4 value = *reinterpret_cast<const u32x4*>(qrow + ks * 16 + half * 8);
    qB[ks] = my_q < S ? value : u32x4{0, 0, 0, 0};
  }

  // Per-lane LDS byte offsets (from the start of a buffer's tile), one per k-step:
  // K operand reads: row 32 t + col, chunk 2 ks + half (rows 32 apart share a swizzle; 32 t RB goes
  // into the immediate offset).
  const uint32_t lds0 = lds_address(lds);
  uint32_t k_off[KS];
  {
    const int kswz = swizzle<D>(col);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) k_off[ks] = lds0 + col * RB + (((2 * ks + half) ^ kswz) << 4);
  }
  // Transposing V reads: lane L = 16g + j supplies row (key) 16 st + 8 r + 4 (g / 2) + j / 4 and
  // columns 16 (g % 2) + 4 (j % 4) of each 32-column tile, so that it receives V[key][32 dt + L % 32]
  // for the keys 16 st + 8 r + 4 (L / 32) + e, e = 0..3 -- the keys its P values cover.  Rows 16 apart
  // share a swizzle (16 st RB goes into the immediate offset).
  uint32_t v_lo[DT], v_hi[DT];
  {
    const int g = lane >> 4, j16 = lane & 15;
    const int tr_row = 4 * (g >> 1) + (j16 >> 2);
    const int tr_col = 16 * (g & 1) + 4 * (j16 & 3);  // element within the 32-column tile
    const int swz_lo = swizzle<D>(tr_row), swz_hi = swizzle<D>(tr_row + 8);
    const int chunk = tr_col >> 3, byte = (tr_col & 7) * 2;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      v_lo[dt] = lds0 + TB + tr_row * RB + (((4 * dt + chunk) ^ swz_lo) << 4) + byte;
      v_hi[dt] = lds0 + TB + (tr_row + 8) * RB + (((4 * dt + chunk) ^ swz_hi) << 4) + byte;
    }
  }

  const float neg_inf = -__builtin_inff();
  f32x16 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f32x16{};
  float m = neg_inf;   // running max of this lane's query (base-2 domain)
  float l_half = 0.f;  // running sum over the keys this half of the wave holds

  auto compute = [&](int kb0, auto buffer) {
    constexpr int BUF = decltype(buffer)::value * 2 * TB;
    // S^T for keys kb0 + 32t + (8i + 4 half + r), r = 0..3, of this lane's query.
    f32x16 s[ST];
#pragma unroll
    for (int t = 0; t < ST; ++t) s[t] = f32x16{};
    // Four k-steps per LDS batch; the tiles' MFMA chains interleave, and each batch's reads are
    // in flight while the previous batch's MFMAs execute.
#pragma unroll
    for (int ks = 0; ks < KS; ks += 4) {
      static_for<ST>([&](auto tile) {
        constexpr int t = decltype(tile)::value;
        u32x4 a[4];
        lds_read_b128_x4<BUF + t * 32 * RB>(a, k_off + ks);
#pragma unroll
        for (int i = 0; i < 4; ++i) s[t] = E::mfma(a[i], qB[ks + i], s[t]);
      });
    }

    // Mask (only the blocks that hold keys past the sequence or past a query of this wave: the test
    // is wave-uniform, so the other blocks skip it), then the block maximum of this lane's query.
    float x[ST][16];
#pragma unroll
    for (int t = 0; t < ST; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) x[t][r] = s[t][r];
    if ((kb0 + BN > S) || (CAUSAL && kb0 + BN - 1 > q_wave)) {
      const int key0 = kb0 + 4 * half;  // key of element (t, r) is key0 + 32 t + 8 (r / 4) + r % 4
      const int limit = CAUSAL ? min(S - 1, my_q) : S - 1;
#pragma unroll
      for (int t = 0; t < ST; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (key0 + 32 * t + 8 * (r >> 2) + (r & 3) > limit) x[t][r] = neg_inf;
    }
    float mx = neg_inf;
#pragma unroll
    for (int t = 0; t < ST; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, x[t][r]);
    mx = max_halves(mx);

    // Online softmax with a lagging reference: probabilities are exp2(x - m) for a reference m that
    // may trail the true running maximum by up to kRescaleSlack, so they stay <= 2^kRescaleSlack
    // (well inside fp16/bf16/fp32 range) and the sum and accumulator use the same reference, which
    // the final division cancels.  m (and with it acc and the sum) moves only when some query's
    // block maximum passes its reference by more than the slack -- in practice in the first blocks.
    const float m_blk = mx * p.scale_log2e;
    if (__builtin_amdgcn_ballot_w64(m_blk > m + kRescaleSlack)) {
      const float m_new = fmaxf(m, m_blk);
      const float alpha = m == neg_inf ? 0.f : fast_exp2(m - m_new);  // 1 where m did not move
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[dt][r] *= alpha;
      l_half *= alpha;
      m = m_new;
    }
    const float m_use = m == neg_inf ? 0.f : m;  // a query with no visible key yet
    float psum = 0.f;
    uint32_t pb[ST][8];  // probabilities in the input dtype, B operands of the PV k-steps
#pragma unroll
    for (int t = 0; t < ST; ++t)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float p0 = fast_exp2(fmaf(x[t][r], p.scale_log2e, -m_use));
        const float p1 = fast_exp2(fmaf(x[t][r + 1], p.scale_log2e, -m_use));
        psum += p0 + p1;
        pb[t][r >> 1] = E::pack(p0, p1);
      }
    l_half += psum;

    // O^T += V^T P^T over the k-steps of 16 keys (k-step st covers keys 16 st .. 16 st + 15).
    static_for<PK>([&](auto step) {
      constexpr int st = decltype(step)::value;
      constexpr int t = st >> 1, sub = st & 1;
      const u32x4 bop = {pb[t][4 * sub], pb[t][4 * sub + 1], pb[t][4 * sub + 2], pb[t][4 * sub + 3]};
      constexpr int OFF = BUF + 16 * st * RB;
      if constexpr (DT == 2) {
        u32x4 a[2];
        lds_read_tr_x2<OFF>(a, v_lo, v_hi);
        acc[0] = E::mfma(a[0], bop, acc[0]);
        acc[1] = E::mfma(a[1], bop, acc[1]);
      } else {
#pragma unroll
        for (int d4 = 0; d4 < DT; d4 += 4) {
          u32x4 a[4];
          lds_read_tr_x4<OFF>(a, v_lo + d4, v_hi + d4);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[d4 + i] = E::mfma(a[i], bop, acc[d4 + i]);
        }
      }
    });
  };

  // One step: wait for this block's tiles (own DMA, then everyone's), start the next block's DMA
  // into the other buffer (free: every wave has finished the previous block), compute.
  auto step = [&](int nb, auto buffer) {
    constexpr int U = decltype(buffer)::value;
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    lds_barrier();
    const int kb0 = nb * BN;
    if (nb + 1 < n_blocks) issue(kb0 + BN, 1 - U);
    if (kb0 + BN > S) {
      // Rows past the sequence hold copies of its last row: zero their V so that a non-finite value
      // there cannot reach other queries through a zero probability.
      constexpr int CHUNKS = TB / 16;
      unsigned char* v_cur = lds + (2 * U + 1) * TB;
      const int first = (S - kb0) * (RB / 16);
#pragma unroll
      for (int c = tid; c < CHUNKS; c += kThreads)
        if (c >= first) *reinterpret_cast<u32x4*>(v_cur + 16 * c) = u32x4{0, 0, 0, 0};
      lds_barrier();
    }
    if (CAUSAL && kb0 > q_wave + 31) return;  // no key of this block is visible to this wave
    compute(kb0, buffer);
  };
  for (int nb = 0; nb < n_blocks; nb += 2) {
    step(nb, Int<0>{});
    if (nb + 1 < n_blocks) step(nb + 1, Int<1>{});
  }

  // Normalise and store: lane holds O^T[32 dt + 8 i + 4 half + r][my_q], r = 0..3 contiguous dims.
  const float l = sum_halves(l_half);
  if (my_q >= S) return;
  const float inv = 1.0f / l;
  uint16_t* orow = p.out + (static_cast<int64_t>(bh) * S + my_q) * D;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d0 = 32 * dt + 8 * i + 4 * half;
      const u32x2 packed = {E::pack(acc[dt][4 * i] * inv, acc[dt][4 * i + 1] * inv),
                            E::pack(acc[dt][4 * i + 2] * inv, acc[dt][4 * i + 3] * inv)};
      *reinterpret_cast<u32x2*>(orow + d0) = packed;
    }
}

// ---------------------------------------------------------------------------------------------
// Host side.
thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buffer[512];
  va_list args;
  va_start(args, fmt);
  vsnprintf(buffer, sizeof(buffer), fmt, args);
  va_end(args);
  g_last_error = buffer;
  return code;
}

// Workgroups resident at once on the 256 CUs for the instantiation a head_dim launches: grids larger
// than this run several rounds and take the XCD-owned grid order.
constexpr int64_t kCus = 256;
int64_t one_round(int64_t head_dim) {
  switch (head_dim) {
    case 64: return Tiling<64, 64>::kOccupancy * kCus;
    case 128: return Tiling<128, 64>::kOccupancy * kCus;
    default: return Tiling<256, 32>::kOccupancy * kCus;
  }
}

template <class E, int D, int BN>
void launch_d(const Params& prm, bool causal, dim3 grid, hipStream_t stream) {
  if (causal)
    hipLaunchKernelGGL((sdpa_fwd_kernel<E, D, BN, true>), grid, dim3(kThreads), 0, stream, prm);
  else
    hipLaunchKernelGGL((sdpa_fwd_kernel<E, D, BN, false>), grid, dim3(kThreads), 0, stream, prm);
}

template <class E>
void launch_e(const Params& prm, int64_t head_dim, bool causal, dim3 grid, hipStream_t stream) {
  if (head_dim == 64)
    launch_d<E, 64, 64>(prm, causal, grid, stream);
  else if (head_dim == 128)
    launch_d<E, 128, 64>(prm, causal, grid, stream);
  else
    launch_d<E, 256, 32>(prm, causal, grid, stream);
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace

extern "C" int rk_sdpa_forward(const void* query, const void* key, const void* value, void* output,
                               int64_t batch, int64_t query_heads, int64_t kv_heads, int64_t sequence,
                               int64_t head_dim, int is_causal, float scale, int dtype, void* stream) {
  if (!query || !key || !value || !output)
    return fail(RK_SDPA_ERR_INVALID_ARGUMENT, "tensor pointers must not be NULL");
  if (dtype != RK_SDPA_DTYPE_FP16 && dtype != RK_SDPA_DTYPE_BF16)
    return fail(RK_SDPA_ERR_INVALID_ARGUMENT, "dtype must be RK_SDPA_DTYPE_FP16 or RK_SDPA_DTYPE_BF16");
  if (batch <= 0 || query_heads <= 0 || kv_heads <= 0 || sequence <= 0)
    return fail(RK_SDPA_ERR_INVALID_ARGUMENT, "tensor dimensions must be positive");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(RK_SDPA_ERR_INVALID_ARGUMENT, "head_dim must be one of 64, 128, 256 (got %lld)",
                static_cast<long long>(head_dim));
  if (query_heads % kv_heads != 0)
    return fail(RK_SDPA_ERR_INVALID_ARGUMENT, "query_heads must be divisible by kv_heads");
  if (is_causal != 0 && is_causal != 1) return fail(RK_SDPA_ERR_INVALID_ARGUMENT, "is_causal must be 0 or 1");
  if (!(scale > 0.0f) || !isfinite(scale))
    return fail(RK_SDPA_ERR_INVALID_ARGUMENT, "scale must be positive and finite");
  if (!aligned16(query) || !aligned16(key) || !aligned16(value) || !aligned16(output))
    return fail(RK_SDPA_ERR_UNSUPPORTED, "query, key, value and output must be 16-byte aligned");
  const int64_t q_blocks = (sequence + kBlockM - 1) / kBlockM;
  if (sequence >= (int64_t{1} << 30) || batch >= (int64_t{1} << 31) || query_heads >= (int64_t{1} << 31) ||
      batch * query_heads > ((int64_t{1} << 62) - 1) / sequence / head_dim)
    return fail(RK_SDPA_ERR_UNSUPPORTED, "shape exceeds the launch limits of this kernel");

  Params prm{};
  prm.q = static_cast<const uint16_t*>(query);
  prm.k = static_cast<const uint16_t*>(key);
  prm.v = static_cast<const uint16_t*>(value);
  prm.out = static_cast<uint16_t*>(output);
  prm.batch = static_cast<int32_t>(batch);
  prm.query_heads = static_cast<int32_t>(query_heads);
  prm.kv_heads = static_cast<int32_t>(kv_heads);
  prm.group = static_cast<int32_t>(query_heads / kv_heads);
  prm.seq = static_cast<int32_t>(sequence);
  prm.q_blocks = static_cast<int32_t>(q_blocks);
  prm.scale_log2e = scale * kLog2e;
  // Grids of one round are resident at once and keep the two-dimensional orders they were tuned
  // with; larger grids take XCD-owned group slices (the one-dimensional grid holds every slice's
  // ceil(q_blocks / S) blocks, padding included, and stays a multiple of 8).
  const int64_t workgroups = batch * query_heads * q_blocks;
  const int64_t groups = batch * kv_heads;
  const int64_t slices = 8 / std::gcd(groups, int64_t{8});
  const int64_t slice_items = (query_heads / kv_heads) * ((q_blocks + slices - 1) / slices);
  const int64_t grid_1d = groups * slices * slice_items;
  const bool sliced = workgroups > one_round(head_dim) && grid_1d < (int64_t{1} << 31);
  // The two-dimensional grid holds (sequence x head, query block) in its y and x extents.
  if (!sliced && (batch * query_heads >= 65536 || q_blocks >= 65536))
    return fail(RK_SDPA_ERR_UNSUPPORTED, "shape exceeds the launch limits of this kernel");
  prm.xcd_slices = sliced ? static_cast<int32_t>(slices) : 0;
  prm.slice_items = static_cast<int32_t>(slice_items);
  const dim3 grid = sliced ? dim3(static_cast<uint32_t>(grid_1d))
                    : is_causal ? dim3(static_cast<uint32_t>(batch * query_heads), static_cast<uint32_t>(q_blocks))
                                : dim3(static_cast<uint32_t>(q_blocks), static_cast<uint32_t>(batch * query_heads));
  hipStream_t hs = static_cast<hipStream_t>(stream);
  if (dtype == RK_SDPA_DTYPE_BF16)
    launch_e<Bf16>(prm, head_dim, is_causal != 0, grid, hs);
  else
    launch_e<Fp16>(prm, head_dim, is_causal != 0, grid, hs);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return fail(RK_SDPA_ERR_LAUNCH, "sdpa launch failed: %s", hipGetErrorString(err));
  return RK_SDPA_OK;
}

extern "C" const char* rk_sdpa_last_error(void) { return g_last_error.c_str(); }

extern "C" const char* rk_sdpa_version(void) { return "rk_sdpa_gfx950 1.0.0 (gfx950, wave64)"; }
