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
//                    each of its 4 waves owns 32 queries and walks the keys in blocks of 64.  Per
//                    block the workgroup stages K and V rows in LDS (row-major, rows padded by 16
//                    bytes); every wave computes S^T = K Q^T with v_mfma_f32_32x32x16 (K rows from
//                    LDS as the A operand, its queries' Q^T held in registers as the B operand), so
//                    each lane owns one query and 16 keys per 32-key tile and the softmax needs one
//                    exchange between the two wave halves; the probabilities, rounded to the input
//                    dtype, are already laid out as the B operand of O^T += V^T P^T, whose A operand
//                    comes from ds_read_b64_tr_b16 transposing reads of the row-major V tile (the
//                    keys of one MFMA k-step are taken in the order the S^T accumulator holds them,
//                    which the transposing read reproduces by the addresses it is given).  The
//                    accumulator is rescaled only when some lane's running maximum moved.  The
//                    register budget is held to three workgroups per CU (at most 170 VGPRs), so one
//                    workgroup's softmax and LDS traffic overlap another's MFMAs; K and V rows go
//                    global -> registers -> LDS at the top of each block rather than being
//                    prefetched a block ahead, which would cost the registers of the third
//                    workgroup (measured: 1.3x slower on the long causal case).  With the causal
//                    mask, blocks past a wave's last query are skipped and the grid runs the longest
//                    query blocks of every head first (1.7x over head-major order on the long
//                    causal case); without it, neighbouring query blocks of one head run together
//                    and share its K and V rows in L2.
//
// Scores are kept in the base-2 domain: p = exp2((q . k) * scale * log2(e) - m), evaluated as one
// fused multiply-add per score; the running maximum m is taken on the raw dot products (scale > 0
// keeps their order) and scaled once per block.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <string>

#include "rk_sdpa.h"

namespace {

constexpr int kWave = 64;
constexpr int kWaves = 4;
constexpr int kThreads = kWave * kWaves;
constexpr int kBlockM = 128;  // queries per workgroup (32 per wave)
constexpr int kBlockN = 64;   // keys per block
constexpr float kLog2e = 1.4426950408889634f;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

struct Bf16 {
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(lo))) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(hi))) << 16);
  }
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   c, 0, 0, 0);
  }
};

struct Fp16 {
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(lo))) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(hi))) << 16);
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
  float scale_log2e;
};

template <class E, int D, bool CAUSAL>
__global__ __launch_bounds__(kThreads, 3) void sdpa_fwd_kernel(Params p) {
  static_assert(D == 64 || D == 128 || D == 256, "head_dim must be 64, 128 or 256");
  constexpr int KS = D / 16;                      // MFMA k-steps of S^T (16 dims each)
  constexpr int DT = D / 32;                      // 32-dim tiles of O^T
  constexpr int ROW = D + 8;                      // LDS row, elements (16-byte pad against bank conflicts)
  constexpr int ROW_CHUNKS = D / 8;               // 16-byte chunks per row
  constexpr int LOADS = kBlockN * ROW_CHUNKS / kThreads;  // chunks per thread per tensor per block
  static_assert(LOADS * kThreads == kBlockN * ROW_CHUNKS, "tile must split evenly over the workgroup");
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[kBlockN * ROW];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[kBlockN * ROW];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int col = lane & 31;

  // Causal: x = (sequence, head), y = query block, longest first (the key range grows with the
  // query block).  Otherwise x = query block, y = (sequence, head).
  const int bh = CAUSAL ? static_cast<int>(blockIdx.x) : static_cast<int>(blockIdx.y);  // b * Hq + hq
  const int qb = CAUSAL ? p.q_blocks - 1 - static_cast<int>(blockIdx.y) : static_cast<int>(blockIdx.x);
  const int b = bh / p.query_heads;
  const int hq = bh - b * p.query_heads;
  const int hkv = hq / p.group;
  const int S = p.seq;
  const int q_wave = qb * kBlockM + wave * 32;  // first query of this wave
  const int my_q = q_wave + col;                // the query this lane owns

  const uint16_t* __restrict__ qrow = p.q + (static_cast<int64_t>(bh) * S + min(my_q, S - 1)) * D;
  const uint16_t* __restrict__ kbase_ptr = p.k + static_cast<int64_t>(b * p.kv_heads + hkv) * S * D;
  const uint16_t* __restrict__ vbase_ptr = p.v + static_cast<int64_t>(b * p.kv_heads + hkv) * S * D;

  // B operand of S^T = K Q^T: column = this lane's query, k-chunk (half) of 8 dims per k-step.
  u32x4 qB[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const u32x4 value = *reinterpret_cast<const u32x4*>(qrow + ks * 16 + half * 8);
    qB[ks] = my_q < S ? value : u32x4{0, 0, 0, 0};
  }

  const int kv_end = CAUSAL ? min(S, (qb + 1) * kBlockM) : S;
  const int n_blocks = (kv_end + kBlockN - 1) / kBlockN;

  // Staging of one K and one V block through registers: chunk c of this thread is row (tid + c*256) / ROW_CHUNKS.
  u32x4 kreg[LOADS], vreg[LOADS];
  auto load_block = [&](int kb) {
#pragma unroll
    for (int c = 0; c < LOADS; ++c) {
      const int chunk = tid + c * kThreads;
      const int row = chunk / ROW_CHUNKS, part = chunk % ROW_CHUNKS;
      const int key = kb * kBlockN + row;
      const int64_t offset = static_cast<int64_t>(min(key, S - 1)) * D + part * 8;  // in bounds; masked later
      kreg[c] = *reinterpret_cast<const u32x4*>(kbase_ptr + offset);
      vreg[c] = key < S ? *reinterpret_cast<const u32x4*>(vbase_ptr + offset) : u32x4{0, 0, 0, 0};
    }
  };
  auto store_block = [&]() {
#pragma unroll
    for (int c = 0; c < LOADS; ++c) {
      const int chunk = tid + c * kThreads;
      const int row = chunk / ROW_CHUNKS, part = chunk % ROW_CHUNKS;
      *reinterpret_cast<u32x4*>(k_lds + row * ROW + part * 8) = kreg[c];
      *reinterpret_cast<u32x4*>(v_lds + row * ROW + part * 8) = vreg[c];
    }
  };

  const float neg_inf = -__builtin_inff();
  f32x16 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f32x16{};
  float m = neg_inf;   // running max of this lane's query (base-2 domain)
  float l_half = 0.f;  // running sum over the keys this half of the wave holds

  // Transposing-read addresses: lane L = 16g + j supplies row (key) 16s + 8r + 4(g/2) + j/4 and
  // columns 16(g%2) + 4(j%4) of each 32-column V tile, so that it receives V[key][32dt + L%32] for
  // the keys 16s + 8r + 4(L/32) + e, e = 0..3 -- the keys its P values cover.
  const int g = lane >> 4, j16 = lane & 15;
  const int tr_row = 4 * (g >> 1) + (j16 >> 2);
  const int tr_col = 16 * (g & 1) + 4 * (j16 & 3);

  for (int nb = 0; nb < n_blocks; ++nb) {
    load_block(nb);
    __syncthreads();  // every wave is done with the previous block's LDS tiles
    store_block();
    __syncthreads();

    const int kb0 = nb * kBlockN;
    if (CAUSAL && kb0 > q_wave + 31) continue;  // no key of this block is visible to this wave

    // S^T for keys kb0 + 32t + (8i + 4 half + r), r = 0..3, of this lane's query.
    f32x16 s[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      s[t] = f32x16{};
      const uint16_t* krow = k_lds + (t * 32 + col) * ROW + half * 8;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(krow + ks * 16);
        s[t] = E::mfma(a, qB[ks], s[t]);
      }
    }

    // Scale, mask, online softmax of this lane's query over the block.
    const bool masked = (kb0 + kBlockN > S) || (CAUSAL && kb0 + kBlockN - 1 > q_wave);
    float x[2][16];
    float mx = neg_inf;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb0 + 32 * t + 8 * (r >> 2) + 4 * half + (r & 3);
        float value = s[t][r];
        if (masked && (key >= S || (CAUSAL && key > my_q))) value = neg_inf;
        x[t][r] = value;
        mx = fmaxf(mx, value);
      }
    mx = max_halves(mx);
    const float m_new = fmaxf(m, mx * p.scale_log2e);
    const float m_use = m_new == neg_inf ? 0.f : m_new;  // a query with no visible key yet
    const float alpha = fast_exp2(m - m_use);            // 0 while m = -inf
    float psum = 0.f;
    uint32_t pb[2][8];  // probabilities in the input dtype, B operands of the four PV k-steps
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float p0 = fast_exp2(fmaf(x[t][r], p.scale_log2e, -m_use));
        const float p1 = fast_exp2(fmaf(x[t][r + 1], p.scale_log2e, -m_use));
        psum += p0 + p1;
        pb[t][r >> 1] = E::pack(p0, p1);
      }
    l_half = l_half * alpha + psum;
    if (__builtin_amdgcn_ballot_w64(m_new != m)) {  // alpha == 1 in every lane leaves acc unchanged
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[dt][r] *= alpha;
    }
    m = m_new;

    // O^T += V^T P^T over four k-steps of 16 keys (k-step st covers keys 16 st .. 16 st + 15).
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int t = st >> 1, sub = st & 1;
      const u32x4 bop = {pb[t][4 * sub], pb[t][4 * sub + 1], pb[t][4 * sub + 2], pb[t][4 * sub + 3]};
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const uint16_t* base = v_lds + (16 * st + tr_row) * ROW + 32 * dt + tr_col;
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base + 8 * ROW));
        const u32x2 lo2 = __builtin_bit_cast(u32x2, lo), hi2 = __builtin_bit_cast(u32x2, hi);
        const u32x4 aop = {lo2[0], lo2[1], hi2[0], hi2[1]};
        acc[dt] = E::mfma(aop, bop, acc[dt]);
      }
    }
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

template <class E, int D>
void launch_d(const Params& prm, bool causal, dim3 grid, hipStream_t stream) {
  if (causal)
    hipLaunchKernelGGL((sdpa_fwd_kernel<E, D, true>), grid, dim3(kThreads), 0, stream, prm);
  else
    hipLaunchKernelGGL((sdpa_fwd_kernel<E, D, false>), grid, dim3(kThreads), 0, stream, prm);
}

template <class E>
void launch_e(const Params& prm, int64_t head_dim, bool causal, dim3 grid, hipStream_t stream) {
  if (head_dim == 64)
    launch_d<E, 64>(prm, causal, grid, stream);
  else if (head_dim == 128)
    launch_d<E, 128>(prm, causal, grid, stream);
  else
    launch_d<E, 256>(prm, causal, grid, stream);
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
  if (batch * query_heads >= 65536 || q_blocks >= 65536 ||
      batch * query_heads * sequence * head_dim >= (int64_t{1} << 62) || sequence >= (int64_t{1} << 30))
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
  const dim3 grid = is_causal ? dim3(static_cast<uint32_t>(batch * query_heads), static_cast<uint32_t>(q_blocks))
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
