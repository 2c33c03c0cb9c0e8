// Block-scaled FP8 linear layer: the o_proj after the attention output gate.
//
// Replaces the reference's triton_block_fp8_linear (qwen3_8/fp8_triton.py:107-183)
// and its GEMM kernel _block_fp8_gemm_kernel (fp8_triton.py:17-98), which
// Qwen3_8FP8Linear._linear_op (qwen3_8/fp8_linear.py:181-201) uses for a
// float8_e4m3fn weight:
//   x_scale = bf16(max(amax|x|, 1e-12) / 448)            dynamic, per tensor
//   xq      = e4m3(clamp(x / x_scale, -448, 448))          round to nearest even
//   out     = bf16(sum_kb (xq[:, kb] w[:, kb]^T) * (x_scale * ws[n / bh, kb / bw]) + bias)
// with fp32 accumulation, kb running over 128-wide slices of K (the weight
// scale blocks are 128 x 128 in the Qwen3 FP8 checkpoints; any block_h and any
// block_w that is a multiple of 128 is accepted here).
//
// Activation quantisation is two HBM-bound passes: act_amax_kernel writes
// per-workgroup maxima of |x| (as bf16 bit patterns, so NaN wins like torch's
// max), act_quant_kernel reduces them, forms x_scale and writes e4m3 rows.
//
// GEMM (fp8_gemm_kernel): out^T tiles D[n][m] = sum_k w[n][k] xq[m][k] with
// v_mfma_f32_16x16x128_f8f6f4 (one instruction covers a whole 128-wide scale
// block).  A workgroup of 2 x WN waves owns 64 WN output columns x 32 MT rows,
// a wave holding 64 columns x 16 MT rows (4 x MT 16x16 tiles): 4 waves
// (128 columns, three K slices in LDS, one wave per SIMD) up to M = 1024,
// 8 waves (256 columns x 256 or 192 rows, two slices in LDS, two waves per
// SIMD) above.  Each MFMA starts from zero and its product is folded into the
// fp32 accumulator with that block's scale, acc += p * s, one FMA per
// accumulator element per 128 of K; a row's folds run between the next row's
// MFMAs, and each row's operand is read from LDS two rows ahead.  Per
// 128-wide K slice the workgroup stages the weight tile (64 WN rows), the
// activation tile (32 MT rows) and the column scales straight from global
// memory into LDS (global_load_lds_dwordx4 / global_load_lds_dword), STAGES - 1
// slices ahead of the MFMAs, a few instructions per row of MFMAs.  Tiles are
// dealt to the XCDs in compact groups (xcd_tile) so that each XCD's L2 serves
// an X or W slice to several of its workgroups.
// Rows are 128 bytes; a row's 16-byte chunk c is stored at chunk
// c ^ swz(row) so the operand reads (16 rows x 16 bytes per 16 lanes) hit 16
// distinct bank groups.  The transposed product makes each lane own four
// consecutive output columns of a row: the epilogue stores 8 bytes per lane.
#include <algorithm>

#include "tf_common.h"
#include "tf_internal.h"

namespace tfa {
namespace {

typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kThreads = 256;          // quantisation kernels
constexpr int kQuantMaxBlocks = TF_FP8_QUANT_WORKSPACE_BYTES / 4;
constexpr float kFp8Max = 448.f;

// ---------------------------------------------------------------- quantisation
struct QuantArgs {
  const uint16_t* x;      // bf16 [rows, cols], row stride xs elements
  int64_t xs;
  uint32_t rows, c8;      // rows, cols / 8
  uint8_t* xq;            // e4m3 [rows, cols], row stride qs bytes
  int64_t qs;
  const uint32_t* partial;   // maxima of |x| bits to reduce (npartial of them)
  uint32_t npartial;
  uint32_t nblocks;
  float* scale_out;
};

__device__ __forceinline__ uint32_t block_max(uint32_t v, uint32_t* red) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, d, kWave));
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  v = red[0];
#pragma unroll
  for (int i = 1; i < kThreads / kWave; ++i) v = max(v, red[i]);
  return v;
}

// Grid-stride loops over 16-byte chunks, kUnroll chunks per trip with their
// loads issued together, so a thread keeps kUnroll loads in flight.
constexpr int kUnroll = 4;

__global__ void __launch_bounds__(kThreads) act_amax_kernel(QuantArgs a, uint32_t* partial) {
  __shared__ uint32_t red[kThreads / kWave];
  const uint32_t n = a.rows * a.c8;
  const uint32_t stride = gridDim.x * kThreads;
  uint32_t m = 0;
  for (uint32_t q0 = blockIdx.x * kThreads + threadIdx.x; q0 < n; q0 += kUnroll * stride) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t q = q0 + u * stride;
      const uint32_t r = q / a.c8, c = q - r * a.c8;
      v[u] = q < n ? ld_nt16(a.x + r * a.xs + 8 * c) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) m = max(m, abs_max8(v[u]));
  }
  m = block_max(m, red);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

__device__ __forceinline__ float sat448(float x) {
  return x != x ? x : fminf(fmaxf(x, -kFp8Max), kFp8Max);
}

__global__ void __launch_bounds__(kThreads) act_quant_kernel(QuantArgs a) {
  __shared__ uint32_t red[kThreads / kWave];
  uint32_t m = 0;
  for (uint32_t i = threadIdx.x; i < a.npartial; i += kThreads) m = max(m, a.partial[i]);
  m = block_max(m, red);
  // amax.clamp(min=1e-12) and amax / 448 on bf16 tensors (fp8_triton.py:128-129):
  // both results are rounded to bf16.  NaN stays NaN.
  float amax = __uint_as_float(m << 16);
  if (m <= 0x7f80u) amax = fmaxf(amax, (float)(__bf16)1e-12f);
  const float scale = (float)(__bf16)(amax / kFp8Max);
  if (blockIdx.x == 0 && threadIdx.x == 0) *a.scale_out = scale;

  const uint32_t n = a.rows * a.c8;
  const uint32_t stride = gridDim.x * kThreads;
  for (uint32_t q0 = blockIdx.x * kThreads + threadIdx.x; q0 < n; q0 += kUnroll * stride) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t q = q0 + u * stride;
      const uint32_t r = q / a.c8, c = q - r * a.c8;
      v[u] = q < n ? ld_nt16(a.x + r * a.xs + 8 * c) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t q = q0 + u * stride;
      if (q >= n) break;
      const uint32_t r = q / a.c8, c = q - r * a.c8;
      u32x2 f;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint32_t lo = __builtin_amdgcn_cvt_pk_fp8_f32(sat448(bf16_lo(v[u][2 * j]) / scale),
                                                            sat448(bf16_hi(v[u][2 * j]) / scale),
                                                            0u, false);
        f[j] = __builtin_amdgcn_cvt_pk_fp8_f32(sat448(bf16_lo(v[u][2 * j + 1]) / scale),
                                               sat448(bf16_hi(v[u][2 * j + 1]) / scale), lo,
                                               true);
      }
      *reinterpret_cast<u32x2*>(a.xq + r * a.qs + 8 * c) = f;
    }
  }
}

// ---------------------------------------------------------------- GEMM
constexpr int kKSlice = 128;          // K per slice = one weight-scale block
constexpr int kSpread = 3;            // staging instructions issued per row of MFMAs
constexpr int kGroupM = 8;            // m-tiles per group of the XCD tile order
constexpr int kMaxSplits = 16;        // split-K factor limit

// A workgroup of 2 x WN waves owns 32 MT activation rows x 64 WN output
// columns; wave (wm, wn) holds rows 16 MT wm .. and columns 64 wn .., i.e.
// 4 x MT 16x16 tiles.  STAGES K slices are resident in LDS, STAGES - 1 staged
// ahead of the MFMAs.
template <int MT, int WN, int STAGES>
struct Tile {
  static constexpr int kWaves = 2 * WN;
  static constexpr int kThreads = kWave * kWaves;
  static constexpr int kBM = 32 * MT;                       // activation rows
  static constexpr int kBN = 64 * WN;                       // output columns
  static constexpr int kXBytes = kBM * kKSlice;
  static constexpr int kWBytes = kBN * kKSlice;
  static constexpr int kSBytes = kWaves * 256;              // 64 scales per wave
  static constexpr int kStage = kXBytes + kWBytes + kSBytes;
  static constexpr int kRowsPerInst = kThreads / 8;         // tile rows per staging instruction
  static constexpr int kXInst = kBM / kRowsPerInst;
  static constexpr int kWInst = kBN / kRowsPerInst;
  static constexpr int kLoads = kXInst + kWInst + 1;        // per thread per slice
  static constexpr int kAhead = STAGES - 1;
  static_assert(kBM % kRowsPerInst == 0 && kBN % kRowsPerInst == 0, "staging rows");
};

struct GemmArgs {
  const uint8_t* xq;      // e4m3 [M, K], row stride xs bytes
  int64_t xs;
  const float* x_scale;   // device scalar
  const uint8_t* w;       // e4m3 [N, K], row stride wrs bytes
  int64_t wrs;
  const float* wsc;       // fp32 block scales (NULL: all 1)
  int64_t sn, sk;         // their strides (elements)
  int32_t bh, bw_slices;  // block_h, block_w / 128
  const uint16_t* bias;   // bf16 [N] or NULL
  uint16_t* out;          // bf16 [M, N], row stride os elements
  int64_t os;
  int32_t M, N, KB, tiles_m;
  int32_t tiles, splits;  // split-K: workgroup = (split, tile), K slices split evenly
  float* part;            // split-K: fp32 [splits, M, N] partial products (NULL: no split)
};

__device__ __forceinline__ int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const lds_void*)p;
}
// global_load_lds_dword{,x4} with a scalar base and a 32-bit per-lane offset:
// lane l's 4 / 16 bytes from sbase + voff land at LDS address M0 + 4 l / 16 l.
// Invisible to the compiler's wait counting: readers wait with an explicit
// s_waitcnt vmcnt and a barrier.
__device__ __forceinline__ void dma4(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
               :: "v"(voff), "s"(sbase), "s"(lds) : "m0");
}
__device__ __forceinline__ void dma16(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(sbase), "s"(lds) : "m0");
}

template <int N>
__device__ __forceinline__ void vm_wait() {
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

// Operand fragment of 16 rows x 128 bytes: lane l holds row l % 16, bytes
// 32 (l / 16) .. + 31 (chunks 2 (l / 16) and 2 (l / 16) + 1, stored swizzled).
// The f8f6f4 MFMA sums over (lane group, byte) pairs in the same way for both
// operands, so any k order shared by the two operands gives the same product.
__device__ __forceinline__ i32x8 frag(const uint8_t* row, int o0, int o1) {
  const u32x4 a = ld_s16(row + o0), b = ld_s16(row + o1);
  i32x8 f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f[j] = (int32_t)a[j];
    f[4 + j] = (int32_t)b[j];
  }
  return f;
}

__device__ __forceinline__ f32x4 mfma_fp8(const i32x8& w, const i32x8& x) {
  // e4m3 x e4m3 (format 0 for both operands), no block exponents: an
  // unscaled v_mfma_f32_16x16x128_f8f6f4 from zero.
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(w, x, f32x4{0.f, 0.f, 0.f, 0.f}, 0,
                                                          0, 0, 0, 0, 0);
}

// Tile order.  Workgroup b of a grid runs on XCD b % 8 (workgroups are dealt to
// the 8 XCDs round-robin), and each XCD takes its workgroups in launch order.
// XCD x gets the contiguous range [x T / 8, (x + 1) T / 8) (rounded) of a
// grouped order in which gm_max consecutive m-tiles share each n-tile, so the
// workgroups one XCD runs at once cover a compact block of tiles (8 m-tiles x
// 4 n-tiles for 32 CUs) whose X and W slices its L2 serves once to all of
// them.  Under split-K (grid = splits x T) the same permutation is applied to
// each split's tiles.
__device__ __forceinline__ void xcd_tile(int b, int tiles, int tiles_m, int gm_max, int* tm,
                                         int* tn) {
  const int x = b & 7, i = b >> 3, q = tiles >> 3, r = tiles & 7;
  const int lin = x * q + min(x, r) + i;
  const int tiles_n = tiles / tiles_m;
  const int group = gm_max * tiles_n;
  const int gid = lin / group, in = lin - gid * group;
  const int gm = min(tiles_m - gid * gm_max, gm_max);
  *tm = gid * gm_max + in % gm;
  *tn = in / gm;
}

// kUni: block_h is a multiple of 64, so the 64 columns of a wave share one
// weight-scale row and the slice's scale is one value per wave.
template <int MT, int WN, int STAGES, bool kUni>
__global__ void __launch_bounds__(2 * kWave * WN)
fp8_gemm_kernel(GemmArgs a) {
  using T = Tile<MT, WN, STAGES>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[STAGES * T::kStage];
  constexpr int kXAhead = kUni ? 2 : 1;   // rows between an operand's read and its use
  const int t = threadIdx.x, w = wave_id(), l = t & 63;
  const int wm = w / WN, wn = w % WN;
  const int split = blockIdx.x / a.tiles;
  int tm_i, tn_i;
  xcd_tile(blockIdx.x % a.tiles, a.tiles, a.tiles_m, kGroupM, &tm_i, &tn_i);
  const int m0 = tm_i * T::kBM;
  const int n0 = tn_i * T::kBN;
  // This workgroup's K slices [kb0, kb0 + KB) (all of them without split-K).
  const int kb0 = (int)((int64_t)a.KB * split / a.splits);
  const int KB = (int)((int64_t)a.KB * (split + 1) / a.splits) - kb0;

  const float xsc = *a.x_scale;
  asm volatile("" :: "v"(xsc));   // land the scale before any staging load is in flight

  // Staging: thread t moves 16-byte chunk t % 8 of row kRowsPerInst i + t / 8
  // of a tile (instruction i), fetched from chunk (t % 8) ^ swz(row) of the
  // source row (swz(row) depends on t only); rows past the matrix repeat its
  // last row.  Byte offsets fit 32 bits.
  const int srow = t >> 3;
  const uint32_t cb = 16 * ((t & 7) ^ swz(srow));
  uint32_t xo[T::kXInst], wo[T::kWInst];
#pragma unroll
  for (int i = 0; i < T::kXInst; ++i)
    xo[i] = (uint32_t)min(m0 + T::kRowsPerInst * i + srow, a.M - 1) * (uint32_t)a.xs + cb;
#pragma unroll
  for (int i = 0; i < T::kWInst; ++i)
    wo[i] = (uint32_t)min(n0 + T::kRowsPerInst * i + srow, a.N - 1) * (uint32_t)a.wrs + cb;
  // Without block scales every lane stages x_scale itself and the staged value
  // is used as is; otherwise the staged weight scale times x_scale.  Wave w
  // stages the scales of columns 64 (w % WN) ..; waves w >= WN stage a copy.
  const bool ones = a.wsc == nullptr;
  const float sfac = ones ? 1.f : xsc;
  const int scol = min(n0 + 64 * wn + l, a.N - 1);
  const uint32_t so = ones ? 0u : (uint32_t)((scol / a.bh) * a.sn) * 4u;
  const uint32_t lds0 = lds_addr(smem);

  // Staging instruction idx of K slice kb into stage st: the X rows
  // (idx < kXInst), the W rows, then the column scales.
  auto issue_one = [&](int kb, int st, int idx) {
    const uint32_t sb = lds0 + st * T::kStage + w * 1024;
    if (idx < T::kXInst) {
      dma16(a.xq + (int64_t)kb * kKSlice, xo[idx], sb + idx * 16 * T::kThreads);
    } else if (idx < T::kXInst + T::kWInst) {
      const int i = idx - T::kXInst;
      dma16(a.w + (int64_t)kb * kKSlice, wo[i], sb + T::kXBytes + i * 16 * T::kThreads);
    } else {
      const float* sbase = ones ? a.x_scale : a.wsc + (int64_t)(kb / a.bw_slices) * a.sk;
      dma4(sbase, so, lds0 + st * T::kStage + T::kXBytes + T::kWBytes + w * 256);
    }
  };
  auto issue = [&](int kb, int st) {
#pragma unroll
    for (int idx = 0; idx < T::kLoads; ++idx) issue_one(kb, st, idx);
  };

  // Fragment reads: row l % 16 of a 16-row tile, chunks 2g and 2g + 1.
  const int rr = l & 15, g = l >> 4;
  const int o0 = 16 * ((2 * g) ^ swz(rr)), o1 = 16 * ((2 * g + 1) ^ swz(rr));
  const int xrow = wm * 16 * MT + rr;   // + 16 tm
  const int wrow = wn * 64 + rr;        // + 16 tn
  const int scol4 = wn * 64 + 4 * g;    // + 16 tn: first of this lane's 4 columns

  f32x4 acc[MT][4];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Slices past the last are never read; their stage is refilled with the last
  // slice so that every step issues (and waits for) the same loads.
#pragma unroll
  for (int i = 0; i < T::kAhead; ++i) issue(kb0 + min(i, KB - 1), i);
  if constexpr (T::kAhead == 2)
    vm_wait<T::kLoads>();
  else
    vm_wait<0>();
  __syncthreads();

  // With one scale per wave, the last row's products of a slice are folded in
  // during the next slice's first row (pl, with that slice's scale in sl);
  // with per-column scales (16 more VGPRs) at the end of the slice.
  f32x4 pl[4], sl[4];
#pragma unroll
  for (int tn = 0; tn < 4; ++tn) pl[tn] = sl[tn] = f32x4{0.f, 0.f, 0.f, 0.f};
  int st = 0;
  for (int j = 0; j < KB; ++j) {
    const int knext = kb0 + min(j + T::kAhead, KB - 1), stn = st == 0 ? STAGES - 1 : st - 1;
    const uint8_t* sp = smem + st * T::kStage;
    const uint8_t* ssp = sp + T::kXBytes + T::kWBytes;
    f32x4 s4[4];
    if constexpr (kUni) {
      const float s1 = sfac * *reinterpret_cast<const float*>(ssp + 4 * (wn * 64));
#pragma unroll
      for (int tn = 0; tn < 4; ++tn) s4[tn] = f32x4{s1, s1, s1, s1};
    } else {
#pragma unroll
      for (int tn = 0; tn < 4; ++tn)
        s4[tn] = sfac * *reinterpret_cast<const f32x4*>(ssp + 4 * (scol4 + 16 * tn));
    }
    i32x8 wf[4], xf[3];
#pragma unroll
    for (int tn = 0; tn < 4; ++tn)
      wf[tn] = frag(sp + T::kXBytes + (wrow + 16 * tn) * kKSlice, o0, o1);
    xf[0] = frag(sp + xrow * kKSlice, o0, o1);
    if constexpr (MT > 1 && kXAhead == 2) xf[1] = frag(sp + (xrow + 16) * kKSlice, o0, o1);
    // Per row tm: up to kSpread staging instructions of slice j + kAhead (the
    // stage they fill was released by the previous step's barrier), the read
    // of row tm + kXAhead's operand, then row tm's four MFMAs, each followed
    // by four FMAs folding row tm - 1's products.  The scheduling barriers
    // keep that order: each MFMA's operand was read kXAhead rows earlier and
    // each product is folded four MFMAs after its own.  (Per-column scales
    // hold 16 more VGPRs per lane, so that variant reads one row ahead.)
    f32x4 p[2][4];
#pragma unroll
    for (int tm = 0; tm < MT; ++tm) {
#pragma unroll
      for (int q = 0; q < kSpread; ++q)
        if (tm * kSpread + q < T::kLoads) issue_one(knext, stn, tm * kSpread + q);
      if (tm == MT - 1)
#pragma unroll
        for (int idx = MT * kSpread; idx < T::kLoads; ++idx) issue_one(knext, stn, idx);
      if (tm + kXAhead < MT)
        xf[(tm + kXAhead) % 3] = frag(sp + (xrow + 16 * (tm + kXAhead)) * kKSlice, o0, o1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int tn = 0; tn < 4; ++tn) {
        p[tm & 1][tn] = mfma_fp8(wf[tn], xf[tm % 3]);
        if (tm > 0)
          acc[tm - 1][tn] += p[(tm - 1) & 1][tn] * s4[tn];
        else if constexpr (kUni)
          acc[MT - 1][tn] += pl[tn] * sl[tn];
      }
      if (tm + kXAhead < MT) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);   // 2 LDS reads
#pragma unroll
      for (int tn = 0; tn < 4; ++tn) {
        __builtin_amdgcn_sched_group_barrier(0x8, 1, 0);   // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x2, 4, 0);   // 4 VALU
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) {
      if constexpr (kUni) {
        pl[tn] = p[(MT - 1) & 1][tn];
        sl[tn] = s4[tn];
      } else {
        acc[MT - 1][tn] += p[(MT - 1) & 1][tn] * s4[tn];
      }
    }
    if constexpr (T::kAhead == 2)
      vm_wait<T::kLoads>();
    else
      vm_wait<0>();
    __syncthreads();
    st = st == STAGES - 1 ? 0 : st + 1;
  }
  vm_wait<0>();   // the refills of the last steps land before the workgroup ends
  if constexpr (kUni) {
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) acc[MT - 1][tn] += pl[tn] * sl[tn];
  }

  // Epilogue: lane holds D[n0 + wn 64 + 16 tn + 4 g + r][m0 + wm 16 MT + 16 tm + rr].
  if (a.part) {   // split-K: fp32 partials, bias and rounding in splitk_reduce_kernel
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) {
      const int n = n0 + scol4 + 16 * tn;
      if (n >= a.N) continue;   // N % 4 == 0: four columns in or out together
#pragma unroll
      for (int tm = 0; tm < MT; ++tm) {
        const int m = m0 + xrow + 16 * tm;
        if (m < a.M)
          *reinterpret_cast<f32x4*>(a.part + ((int64_t)split * a.M + m) * a.N + n) = acc[tm][tn];
      }
    }
    return;
  }
#pragma unroll
  for (int tn = 0; tn < 4; ++tn) {
    const int n = n0 + scol4 + 16 * tn;
    float b[4] = {0.f, 0.f, 0.f, 0.f};
    if (a.bias) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (n + r < a.N) b[r] = __uint_as_float((uint32_t)a.bias[n + r] << 16);
    }
#pragma unroll
    for (int tm = 0; tm < MT; ++tm) {
      const int m = m0 + xrow + 16 * tm;
      if (m >= a.M) continue;
      const f32x4 v = acc[tm][tn];
      uint16_t* o = a.out + (int64_t)m * a.os + n;
      if (n + 3 < a.N) {
        u32x2 pk;
        pk[0] = pack_bf16(v[0] + b[0], v[1] + b[1]);
        pk[1] = pack_bf16(v[2] + b[2], v[3] + b[3]);
        *reinterpret_cast<u32x2*>(o) = pk;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < a.N) o[r] = (uint16_t)(pack_bf16(v[r] + b[r], 0.f) & 0xffffu);
      }
    }
  }
}

// out = bf16(sum over splits of the fp32 partials (in split order) + bias);
// one thread per four consecutive columns (N % 4 == 0).  Every partial is
// loaded before the first add, so the loads' latencies overlap.
__global__ void __launch_bounds__(kThreads) splitk_reduce_kernel(GemmArgs a) {
  const int64_t e = 4 * ((int64_t)blockIdx.x * kThreads + threadIdx.x);
  const int64_t mn = (int64_t)a.M * a.N;
  if (e >= mn) return;
  const int m = (int)(e / a.N), n = (int)(e - (int64_t)m * a.N);
  f32x4 p[kMaxSplits];
#pragma unroll
  for (int sp = 0; sp < kMaxSplits; ++sp)
    if (sp < a.splits) p[sp] = *reinterpret_cast<const f32x4*>(a.part + sp * mn + e);
  f32x4 v = p[0];
#pragma unroll
  for (int sp = 1; sp < kMaxSplits; ++sp)
    if (sp < a.splits) v += p[sp];
  float b[4] = {0.f, 0.f, 0.f, 0.f};
  if (a.bias) {
#pragma unroll
    for (int r = 0; r < 4; ++r) b[r] = __uint_as_float((uint32_t)a.bias[n + r] << 16);
  }
  u32x2 pk;
  pk[0] = pack_bf16(v[0] + b[0], v[1] + b[1]);
  pk[1] = pack_bf16(v[2] + b[2], v[3] + b[3]);
  *reinterpret_cast<u32x2*>(a.out + (int64_t)m * a.os + n) = pk;
}

// Tile shape by M: (MT, WN, STAGES).
struct Shape {
  int mt, wn;
};
Shape gemm_shape(int64_t m, int64_t n) {
  if (m <= 32) return {1, 2};
  if (m <= 64) return {2, 2};
  if (m <= 128) return {4, 2};
  if (m <= 1024) return {8, 2};
  // 8 waves, 256 columns, 2 waves per SIMD: 256 or 192 rows, whichever ends
  // sooner when the tiles run in rounds of one per CU; a 192-row tile takes
  // 0.8 of a 256-row one (measured at m = 4096, 8320, 21938: 192 rows win at
  // 4096, 256 at the other two).
  const int64_t cus = device_cu_count(), tn = (n + 255) / 256;
  const int64_t r256 = ((m + 255) / 256 * tn + cus - 1) / cus;
  const int64_t r192 = ((m + 191) / 192 * tn + cus - 1) / cus;
  return 5 * r256 <= 4 * r192 ? Shape{8, 4} : Shape{6, 4};
}

// Split-K factor: when the output tiles alone leave most CUs idle (M up to 512,
// the weight-streaming regime), K is split so that the workgroups fill the
// device's CUs (256 on MI355X) in one round (320 workgroups, one and a quarter
// rounds, took 1.4 times as long at M = 64).
int gemm_splits(int64_t m, int64_t n, int64_t k) {
  const Shape sh = gemm_shape(m, n);
  if (m > 512 || n % 4) return 1;
  const int64_t cus = device_cu_count();
  const int64_t tiles = ((m + 32 * sh.mt - 1) / (32 * sh.mt)) * ((n + 64 * sh.wn - 1) / (64 * sh.wn));
  const int64_t kb = k / kKSlice;
  if (tiles >= cus / 2 || kb < 4) return 1;
  return (int)std::max<int64_t>(1, std::min<int64_t>({kb / 2, cus / tiles, kMaxSplits}));
}

template <int MT, int WN, int STAGES>
void launch_gemm(const GemmArgs& a, hipStream_t stream) {
  using T = Tile<MT, WN, STAGES>;
  GemmArgs b = a;
  b.tiles_m = (a.M + T::kBM - 1) / T::kBM;
  const int tiles_n = (a.N + T::kBN - 1) / T::kBN;
  b.tiles = b.tiles_m * tiles_n;
  const dim3 grid(b.tiles * b.splits), block(T::kThreads);
  if (a.wsc == nullptr || a.bh % 64 == 0)
    hipLaunchKernelGGL((fp8_gemm_kernel<MT, WN, STAGES, true>), grid, block, 0, stream, b);
  else
    hipLaunchKernelGGL((fp8_gemm_kernel<MT, WN, STAGES, false>), grid, block, 0, stream, b);
  if (b.part) {
    const int64_t groups = ((int64_t)a.M * a.N / 4 + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((uint32_t)groups), dim3(kThreads), 0, stream, b);
  }
}

// Validates the arguments both quantisation entry points share and fills a.
int32_t quant_setup(const char* fn, const void* x, int32_t x_dtype, int64_t rows, int64_t cols,
                    int64_t x_row_stride, void* xq, int64_t xq_row_stride, float* x_scale,
                    QuantArgs* a) {
  if (x_dtype != TF_DTYPE_BF16)
    return fail(TF_ERR_UNSUPPORTED, "%s: x must be bf16 (dtype %d)", fn, x_dtype);
  if (rows < 0 || cols <= 0 || cols % 8 || x_row_stride < cols || xq_row_stride < cols)
    return fail(TF_ERR_INVALID, "%s: rows=%lld cols=%lld (a multiple of 8) strides %lld/%lld",
                fn, (long long)rows, (long long)cols, (long long)x_row_stride,
                (long long)xq_row_stride);
  if (x_row_stride % 8 || xq_row_stride % 8)
    return fail(TF_ERR_INVALID, "%s: row strides must be multiples of 8", fn);
  if (rows * (cols / 8) > (int64_t)UINT32_MAX / 2 || rows * x_row_stride > INT64_MAX / 4)
    return fail(TF_ERR_UNSUPPORTED, "%s: %lld x %lld is too large", fn, (long long)rows,
                (long long)cols);
  if ((rows > 0 && (!x || !xq)) || !x_scale)
    return fail(TF_ERR_INVALID, "%s: null pointer", fn);
  if (!aligned16(x) || !aligned8(xq))
    return fail(TF_ERR_INVALID, "%s: x must be 16-byte and xq 8-byte aligned", fn);
  a->x = static_cast<const uint16_t*>(x);
  a->xs = x_row_stride;
  a->rows = (uint32_t)rows;
  a->c8 = (uint32_t)(cols / 8);
  a->xq = static_cast<uint8_t*>(xq);
  a->qs = xq_row_stride;
  a->scale_out = x_scale;
  // ~2 chunks (32 B of x) per thread, at most kQuantMaxBlocks workgroups:
  // small inputs spread over many CUs (one round of loads each), large ones
  // loop with kUnroll loads in flight per thread
  const int64_t chunks = rows * (cols / 8);
  const int64_t want = (chunks + 2 * kThreads - 1) / (2 * kThreads);
  a->nblocks = (uint32_t)std::max<int64_t>(1, std::min<int64_t>(want, kQuantMaxBlocks));
  return TF_OK;
}

}  // namespace
}  // namespace tfa

extern "C" {

int32_t tf_fp8_act_quant(const void* x, int32_t x_dtype, int64_t rows, int64_t cols,
                         int64_t x_row_stride, void* xq, int64_t xq_row_stride,
                         float* x_scale, void* workspace, int64_t workspace_bytes,
                         tf_stream_t stream) {
  using namespace tfa;
  clear_error();
  QuantArgs a;
  const int32_t rc = quant_setup("fp8_act_quant", x, x_dtype, rows, cols, x_row_stride, xq,
                                 xq_row_stride, x_scale, &a);
  if (rc != TF_OK) return rc;
  if (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 3u))
    return fail(TF_ERR_INVALID, "fp8_act_quant: workspace must be 4-byte aligned");
  if (workspace_bytes < TF_FP8_QUANT_WORKSPACE_BYTES)
    return fail(TF_ERR_INVALID, "fp8_act_quant: workspace of %lld bytes (needs %d)",
                (long long)workspace_bytes, TF_FP8_QUANT_WORKSPACE_BYTES);
  uint32_t* partial = static_cast<uint32_t*>(workspace);
  a.partial = partial;
  a.npartial = a.nblocks;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(act_amax_kernel, dim3(a.nblocks), dim3(kThreads), 0, s, a, partial);
  hipLaunchKernelGGL(act_quant_kernel, dim3(a.nblocks), dim3(kThreads), 0, s, a);
  return launch_status("tf_fp8_act_quant launch");
}

int32_t tf_fp8_act_quant_amax(const void* x, int32_t x_dtype, int64_t rows, int64_t cols,
                              int64_t x_row_stride, void* xq, int64_t xq_row_stride,
                              float* x_scale, const uint32_t* amax_bits, tf_stream_t stream) {
  using namespace tfa;
  clear_error();
  QuantArgs a;
  const int32_t rc = quant_setup("fp8_act_quant_amax", x, x_dtype, rows, cols, x_row_stride,
                                 xq, xq_row_stride, x_scale, &a);
  if (rc != TF_OK) return rc;
  if (!amax_bits || (reinterpret_cast<uintptr_t>(amax_bits) & 3u))
    return fail(TF_ERR_INVALID, "fp8_act_quant_amax: amax_bits must be a 4-byte aligned "
                "device pointer");
  a.partial = amax_bits;
  a.npartial = 1;
  hipLaunchKernelGGL(act_quant_kernel, dim3(a.nblocks), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), a);
  return launch_status("tf_fp8_act_quant_amax launch");
}

int32_t tf_fp8_block_gemm(const void* xq, int64_t xq_row_stride, const float* x_scale,
                          const void* w, int64_t w_row_stride, const float* w_scale,
                          int64_t w_scale_row_stride, int64_t w_scale_col_stride,
                          int32_t block_h, int32_t block_w, const void* bias, int64_t m,
                          int64_t n, int64_t k, void* out, int64_t out_row_stride,
                          void* workspace, int64_t workspace_bytes, tf_stream_t stream) {
  using namespace tfa;
  clear_error();
  if (m < 0 || n <= 0 || k <= 0 || k % kKSlice)
    return fail(TF_ERR_INVALID, "fp8_block_gemm: m=%lld n=%lld k=%lld (k a multiple of 128)",
                (long long)m, (long long)n, (long long)k);
  if (m > INT32_MAX / 2 || n > INT32_MAX / 2 || k > INT32_MAX / 2)
    return fail(TF_ERR_UNSUPPORTED, "fp8_block_gemm: dimensions too large");
  if (xq_row_stride < k || w_row_stride < k || out_row_stride < n || xq_row_stride % 16 ||
      w_row_stride % 16 || out_row_stride % 4)
    return fail(TF_ERR_INVALID,
                "fp8_block_gemm: row strides %lld/%lld/%lld (fp8 rows 16-byte, out rows "
                "8-byte multiples)",
                (long long)xq_row_stride, (long long)w_row_stride, (long long)out_row_stride);
  if (!w || !x_scale || (m > 0 && (!xq || !out)))
    return fail(TF_ERR_INVALID, "fp8_block_gemm: null pointer");
  if (!aligned16(xq) || !aligned16(w) || !aligned8(out) ||
      (reinterpret_cast<uintptr_t>(bias) & 1u))
    return fail(TF_ERR_INVALID, "fp8_block_gemm: xq / w 16-byte, out 8-byte aligned");
  if (w_scale && (block_h <= 0 || block_w <= 0 || block_w % kKSlice))
    return fail(TF_ERR_UNSUPPORTED,
                "fp8_block_gemm: block_h=%d block_w=%d (block_w a multiple of 128)", block_h,
                block_w);
  if (m == 0) return TF_OK;
  if ((m - 1) * xq_row_stride + k > (int64_t)UINT32_MAX ||
      (n - 1) * w_row_stride + k > (int64_t)UINT32_MAX ||
      (w_scale && ((n - 1) / block_h) * w_scale_row_stride > (int64_t)(UINT32_MAX / 4)))
    return fail(TF_ERR_UNSUPPORTED, "fp8_block_gemm: xq, w or w_scale spans more than 4 GiB");
  GemmArgs a;
  a.xq = static_cast<const uint8_t*>(xq);
  a.xs = xq_row_stride;
  a.x_scale = x_scale;
  a.w = static_cast<const uint8_t*>(w);
  a.wrs = w_row_stride;
  a.wsc = w_scale;
  a.sn = w_scale_row_stride;
  a.sk = w_scale_col_stride;
  a.bh = w_scale ? block_h : 1;
  a.bw_slices = w_scale ? block_w / kKSlice : 1;
  a.bias = static_cast<const uint16_t*>(bias);
  a.out = static_cast<uint16_t*>(out);
  a.os = out_row_stride;
  a.M = (int32_t)m;
  a.N = (int32_t)n;
  a.KB = (int32_t)(k / kKSlice);
  a.tiles_m = 0;
  a.tiles = 0;
  a.splits = 1;
  a.part = nullptr;
  // Split-K when a large enough 16-byte aligned workspace comes with the call;
  // otherwise (or when it does not pay) one workgroup per output tile.
  const int splits = gemm_splits(m, n, k);
  if (splits > 1 && workspace && !(reinterpret_cast<uintptr_t>(workspace) & 15u) &&
      workspace_bytes >= (int64_t)splits * m * n * 4) {
    a.splits = splits;
    a.part = static_cast<float*>(workspace);
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const Shape sh = gemm_shape(m, n);
  if (sh.mt == 1)
    launch_gemm<1, 2, 3>(a, s);
  else if (sh.mt == 2)
    launch_gemm<2, 2, 3>(a, s);
  else if (sh.mt == 4)
    launch_gemm<4, 2, 3>(a, s);
  else if (sh.wn == 2)
    launch_gemm<8, 2, 3>(a, s);
  else if (sh.mt == 6)
    launch_gemm<6, 4, 2>(a, s);
  else
    launch_gemm<8, 4, 2>(a, s);
  return launch_status("tf_fp8_block_gemm launch");
}

int64_t tf_fp8_block_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  using namespace tfa;
  clear_error();
  if (m < 0 || n <= 0 || k <= 0 || k % kKSlice)
    return fail(TF_ERR_INVALID, "fp8_block_gemm_workspace_bytes: m=%lld n=%lld k=%lld",
                (long long)m, (long long)n, (long long)k);
  const int splits = gemm_splits(m, n, k);
  return splits > 1 ? (int64_t)splits * m * n * 4 : 0;
}

}  // extern "C"
