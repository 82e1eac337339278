// gemm_int4.hip — MatMulNBits int4 GEMM for gfx950 (fp16 MFMA, f32 accumulate).
//
// Computes out[t][n] = sum_b scale[n][b] * sum_{k in b} x[t][k] * (q[n][k] - zp[n][b]) + bias[n]
// over the ONNX MatMulNBits layout (uint4 packed two per byte along K, low
// nibble first; fp16 scales [N][K/32]; packed uint4 zero-points
// [N][ceil(K/64)], even block in the low nibble) — the semantics of
// matmulInt4BlockImpl, packages/textsift/src/zig/wasm_exports.zig:560-707.
//
// Mapping to CDNA4:
//  * One v_mfma_f32_16x16x32_f16 K-step is exactly one 32-wide quant block.
//    Weights enter the MFMA as the exact small integers (q - zp) in fp16, so
//    every product is exact; the block's f32 partial sum is then scaled with
//    one fmaf per accumulator, as the reference scales per block.
//  * The GEMM is computed transposed (D = W . X^T): the MFMA's M dimension
//    runs over weight rows, so each lane ends up holding 4 consecutive output
//    columns of one token. That makes the epilogues lane-local: RoPE pairs
//    (2p, 2p+1) and SwiGLU's interleaved (gate, up) columns sit in one lane,
//    and stores are 8-16 byte vectors.
//  * f32 activations (the WASM path feeds f32 to Q/K/V, router and experts,
//    browser/inference/block.ts:126-176) enter as an exact fp16 hi + lo pair
//    (two MFMAs into the same block partial), carrying 22 significant bits.
//  * Workgroup tile: 128 weight rows x BT tokens, K staged 64 at a time
//    through LDS (W dequantised once per workgroup, X split once), global
//    loads for the next stage issued before the current stage's MFMAs.
//  * Workgroup ids are remapped so each XCD walks a contiguous range of
//    (token tile, n tile) pairs: the n tiles of one token tile share an L2.
//  * Grouped mode: tiles come from a device list of (expert, row0, rows)
//    built by the MoE routing kernels; weights are offset per expert and
//    activation rows may be gathered through row_map.
#include "common.h"
#include "epilogue.h"
#include "pfhip_internal.h"

namespace pf {

namespace {

constexpr int BN = 128;         // weight rows (output columns) per workgroup
constexpr int BK = 64;          // K per LDS stage = two quant blocks
constexpr int LDW = BK + 8;     // padded LDS row (halves)

// (1024 + a, 1024 + b) - (1024 + zp, 1024 + zp) on packed fp16: exact.
// Scalars only: __builtin_bit_cast applied to an ext-vector element (r.y)
// is lowered by this clang as a cast of the previously assigned element.
__device__ __forceinline__ uint32_t sub_zp(uint32_t v, h2_t off) {
  const h2_t h = __builtin_bit_cast(h2_t, v) - off;
  return __builtin_bit_cast(uint32_t, h);
}

// 8 nibbles of one dword -> 8 exact fp16 values (q - zp), natural k order.
__device__ __forceinline__ u4_t dequant8(uint32_t w, uint32_t zp_pair) {
  const uint32_t lo = w & 0x0F0F0F0Fu;          // k0 k2 k4 k6
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;   // k1 k3 k5 k7
  const h2_t off = __builtin_bit_cast(h2_t, zp_pair);  // (1024+zp, 1024+zp)
  const uint32_t p0 = __builtin_amdgcn_perm(hi, lo, 0x0C040C00u) | 0x64006400u;  // 1024+k0, 1024+k1
  const uint32_t p1 = __builtin_amdgcn_perm(hi, lo, 0x0C050C01u) | 0x64006400u;
  const uint32_t p2 = __builtin_amdgcn_perm(hi, lo, 0x0C060C02u) | 0x64006400u;
  const uint32_t p3 = __builtin_amdgcn_perm(hi, lo, 0x0C070C03u) | 0x64006400u;
  return u4_t{sub_zp(p0, off), sub_zp(p1, off), sub_zp(p2, off), sub_zp(p3, off)};
}

__device__ __forceinline__ int xcd_remap(int bid, int total) {
  const int xcd = bid & 7, idx = bid >> 3;
  const int per = total >> 3, rem = total & 7;
  return xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
}

template <int BT, bool SPLIT, Epi EPI, bool GROUPED>
__global__ __launch_bounds__(256) void k_gemm_int4(GemmArgs p) {
  constexpr int NPL = SPLIT ? 2 : 1;
  constexpr int WT = BT / 2;   // tokens per wave
  constexpr int WN = BN / 2;   // weight rows per wave
  constexpr int TI = WN / 16;  // n sub-tiles per wave
  constexpr int TJ = WT / 16;  // token sub-tiles per wave
  // X loader geometry: 8 x 16-byte chunks per row per plane per stage
  constexpr int XCH = 8;
  constexpr int XRP = 256 / XCH;                 // rows per pass
  constexpr int XPASS = BT / XRP;                // passes

  __shared__ __attribute__((aligned(16))) _Float16 Wl[BN * LDW];
  __shared__ __attribute__((aligned(16))) float Sl[2 * BN];
  __shared__ __attribute__((aligned(16))) _Float16 Xl[NPL * BT * LDW];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wn = (wave & 1) * WN;
  const int wt = (wave >> 1) * WT;
  const int l16 = lane & 15, lg = lane >> 4;

  const int n_tiles = (p.N + BN - 1) / BN;
  // grouped: the XCD remap over the workgroups that have tiles (the grid
  // covers the largest possible tile list)
  int active = (int)gridDim.x;
  if constexpr (GROUPED) {
    active = min(active, *p.num_tiles * n_tiles);
    if ((int)blockIdx.x >= active) return;
  }
  const int bid = xcd_remap(blockIdx.x, active);
  const int nt = bid % n_tiles;
  const int tt = bid / n_tiles;
  int expert = 0, row0, rows;
  if constexpr (GROUPED) {
    if (tt >= *p.num_tiles) return;
    const int4 ti = reinterpret_cast<const int4*>(p.tiles)[tt];
    expert = ti.x;
    row0 = ti.y;
    rows = ti.z;
  } else {
    row0 = tt * BT;
    rows = min(BT, p.M - row0);
    if (rows <= 0) return;
  }
  const int n0 = nt * BN;
  const int K = p.K;
  const int nb = K >> 5;
  const int zstride = (nb + 1) >> 1;
  const uint8_t* __restrict__ W = p.w + (size_t)expert * p.w_gs;
  const uint16_t* __restrict__ WS = p.ws + (size_t)expert * p.ws_gs;
  const uint8_t* __restrict__ WZ = p.wz ? p.wz + (size_t)expert * p.wz_gs : nullptr;

  // ---- loader roles
  const int wr = tid >> 1, wb = tid & 1;       // W: row, block within stage
  const int wrow = n0 + wr;
  const bool w_ok = wrow < p.N;
  const uint8_t* wsrc = W + (size_t)wrow * (K >> 1);

  const int xr = tid / XCH, xc = tid % XCH;
  int xoff[XPASS];                              // element offset of each X row, -1 = zero row
#pragma unroll
  for (int i = 0; i < XPASS; ++i) {
    const int r = xr + i * XRP;
    if (r < rows) {
      const int lr = row0 + r;
      const int g = p.row_map ? p.row_map[lr] : lr;
      xoff[i] = g * p.ldx;
    } else {
      xoff[i] = -1;
    }
  }

  // ---- prefetch registers: raw bytes only. Nothing loaded here is consumed
  // before store_stage, so the next stage's loads stay in flight across the
  // current stage's MFMAs (decoding a scale or zero-point here would make the
  // compiler wait for the load right away).
  u4_t wreg;
  uint32_t sraw;   // fp16 scale bits
  uint32_t zraw;   // zero-point byte (nibble selected in store_stage)
  bool wvalid;
  u4_t xreg[NPL][XPASS];
  const uint16_t* __restrict__ xhi = static_cast<const uint16_t*>(p.x);
  const uint16_t* __restrict__ xlo = p.x_lo;
  int kb_cur = 0;

  auto load_stage = [&](int s) {
    const int kb = s * 2 + wb;
    kb_cur = kb;
    wvalid = w_ok && kb < nb;
    if (wvalid) {
      wreg = *reinterpret_cast<const u4_t*>(wsrc + kb * 16);
      sraw = WS[(size_t)wrow * nb + kb];
      zraw = WZ ? (uint32_t)WZ[(size_t)wrow * zstride + (kb >> 1)] : 0u;
    }
#pragma unroll
    for (int i = 0; i < XPASS; ++i) {
      const int k = s * BK + xc * 8;
      if (xoff[i] >= 0 && k < K) {
        xreg[0][i] = *reinterpret_cast<const u4_t*>(xhi + xoff[i] + k);
        if constexpr (SPLIT) xreg[1][i] = *reinterpret_cast<const u4_t*>(xlo + xoff[i] + k);
      } else {
        xreg[0][i] = u4_t{0u, 0u, 0u, 0u};
        if constexpr (SPLIT) xreg[1][i] = u4_t{0u, 0u, 0u, 0u};
      }
    }
  };

  auto store_stage = [&]() {
    // W: 32 nibbles -> 32 exact fp16 at Wl[wr][wb*32 ...]; invalid rows /
    // blocks store q = 8 with zp = 8 (exact zeros) and scale 0.
    u4_t wq = u4_t{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};
    uint32_t zp = 8;
    float sc = 0.0f;
    if (wvalid) {
      wq = wreg;
      sc = wasm_h2f((uint16_t)sraw);
      zp = WZ ? ((kb_cur & 1) ? (zraw >> 4) : (zraw & 0xFu)) : 0u;
    }
    const uint32_t hz = 0x6400u + zp;  // fp16 bits of 1024 + zp
    const uint32_t zreg = hz | (hz << 16);
    u4_t* wdst = reinterpret_cast<u4_t*>(&Wl[wr * LDW + wb * 32]);
    wdst[0] = dequant8(wq.x, zreg);
    wdst[1] = dequant8(wq.y, zreg);
    wdst[2] = dequant8(wq.z, zreg);
    wdst[3] = dequant8(wq.w, zreg);
    Sl[wb * BN + wr] = sc;
#pragma unroll
    for (int i = 0; i < XPASS; ++i) {
      const int r = xr + i * XRP;
#pragma unroll
      for (int pl = 0; pl < NPL; ++pl)
        *reinterpret_cast<u4_t*>(&Xl[pl * BT * LDW + r * LDW + xc * 8]) = xreg[pl][i];
    }
  };

  f4_t acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

  const int S = (nb + 1) >> 1;
  load_stage(0);
  for (int s = 0; s < S; ++s) {
    if (s > 0) __syncthreads();
    store_stage();
    __syncthreads();
    if (s + 1 < S) load_stage(s + 1);
    const int nblk = min(2, nb - 2 * s);
    for (int b = 0; b < nblk; ++b) {
      h8_t wf[TI], xh[TJ], xl[TJ];
      f4_t sc[TI];
#pragma unroll
      for (int i = 0; i < TI; ++i) {
        wf[i] = *reinterpret_cast<const h8_t*>(&Wl[(wn + 16 * i + l16) * LDW + b * 32 + 8 * lg]);
        sc[i] = *reinterpret_cast<const f4_t*>(&Sl[b * BN + wn + 16 * i + 4 * lg]);
      }
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        xh[j] = *reinterpret_cast<const h8_t*>(&Xl[(wt + 16 * j + l16) * LDW + b * 32 + 8 * lg]);
        if constexpr (SPLIT)
          xl[j] = *reinterpret_cast<const h8_t*>(&Xl[BT * LDW + (wt + 16 * j + l16) * LDW + b * 32 + 8 * lg]);
      }
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
          f4_t t = mfma16x16x32(wf[i], xh[j], f4_t{0.f, 0.f, 0.f, 0.f});
          if constexpr (SPLIT) t = mfma16x16x32(wf[i], xl[j], t);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[i][j][r] = fmaf(t[r], sc[i][r], acc[i][j][r]);
        }
    }
  }

  // ---- epilogue: lane holds out[token = wt+16j+l16][n = wn+16i+4lg+r]
  const uint16_t* __restrict__ BIAS = p.bias ? p.bias + (size_t)expert * p.bias_gs : nullptr;
#pragma unroll
  for (int i = 0; i < TI; ++i) {
    const int n = n0 + wn + 16 * i + 4 * lg;
    float bv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) bv[r] = (BIAS && n + r < p.N) ? wasm_h2f(BIAS[n + r]) : 0.0f;
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int lt = wt + 16 * j + l16;
      if (lt >= rows) continue;
      const size_t orow = (size_t)(row0 + lt);
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = acc[i][j][r] + bv[r];
      int pos = 0;
      if constexpr (EPI == Epi::ROPE_F16) pos = (int)((uint32_t)orow % (uint32_t)p.seq_len);  // rows < 2^31
      store_out<EPI>(p, orow, n, v, pos);
    }
  }
}

template <int BT, bool SPLIT, Epi EPI, bool GROUPED>
void launch(pfhip_backend* b, const GemmArgs& a, const char* name) {
  const int n_tiles = (a.N + BN - 1) / BN;
  const int t_tiles = GROUPED ? a.max_tiles : (a.M + BT - 1) / BT;
  const long grid = (long)n_tiles * t_tiles;
  if (grid == 0) return;
  PF_CHECK(grid < (1L << 31), "gemm_int4: grid too large");
  ProfScope ps(b, name);
  hipLaunchKernelGGL((k_gemm_int4<BT, SPLIT, EPI, GROUPED>), dim3((unsigned)grid), dim3(256), 0, b->stream, a);
  PF_HIP(hipGetLastError());
}

template <int BT, bool SPLIT, bool GROUPED>
void dispatch_epi(pfhip_backend* b, const GemmArgs& a, Epi epi, const char* name) {
  switch (epi) {
    case Epi::F16: return launch<BT, SPLIT, Epi::F16, GROUPED>(b, a, name);
    case Epi::F32: return launch<BT, SPLIT, Epi::F32, GROUPED>(b, a, name);
    case Epi::ROPE_F16: return launch<BT, SPLIT, Epi::ROPE_F16, GROUPED>(b, a, name);
    case Epi::SWIGLU_SPLIT: return launch<BT, SPLIT, Epi::SWIGLU_SPLIT, GROUPED>(b, a, name);
    case Epi::SWIGLU_F16: return launch<BT, SPLIT, Epi::SWIGLU_F16, GROUPED>(b, a, name);
    case Epi::F32_TOPK: break;
  }
  throw Error("gemm_int4: unsupported epilogue");
}

}  // namespace

void gemm_int4(pfhip_backend* b, const GemmArgs& a, XKind xk, Epi epi, bool grouped, int tile_t,
               const char* prof_name) {
  PF_CHECK(a.K > 0 && a.K % 32 == 0, "gemm_int4: K must be a positive multiple of 32");
  PF_CHECK(a.N > 0, "gemm_int4: N must be positive");
  PF_CHECK(a.x && a.w && a.ws && a.out, "gemm_int4: null operand");
  PF_CHECK(a.ldx % 8 == 0 && a.K % 8 == 0, "gemm_int4: activation row stride must allow 16-byte loads");
  PF_CHECK((reinterpret_cast<uintptr_t>(a.x) & 15) == 0 && (reinterpret_cast<uintptr_t>(a.w) & 15) == 0,
           "gemm_int4: activations and weights must be 16-byte aligned");
  if (xk == XKind::SPLIT)
    PF_CHECK(a.x_lo && (reinterpret_cast<uintptr_t>(a.x_lo) & 15) == 0, "gemm_int4: SPLIT needs an aligned lo plane");
  PF_CHECK(a.K / 2 % 16 == 0, "gemm_int4: packed weight rows must be 16-byte multiples");
  if (epi == Epi::SWIGLU_SPLIT || epi == Epi::SWIGLU_F16) PF_CHECK(a.N % 4 == 0, "gemm_int4: SwiGLU needs N % 4 == 0");
  if (epi == Epi::SWIGLU_SPLIT) PF_CHECK(a.out_lo, "gemm_int4: SWIGLU_SPLIT needs an output lo plane");
  if (epi == Epi::ROPE_F16)
    PF_CHECK(a.rope_cos && a.rope_sin && a.seq_len > 0 && a.rope_cols % 64 == 0,
             "gemm_int4: RoPE epilogue needs tables, seq_len and head-aligned rope_cols");
  if (epi == Epi::ROPE_F16) PF_CHECK(!grouped && (long)a.M < (1L << 31), "RoPE epilogue: dense rows below 2^31");
  if (grouped) PF_CHECK(a.tiles && a.num_tiles && a.max_tiles > 0, "gemm_int4: grouped mode needs a tile list");
  else PF_CHECK(a.M >= 0, "gemm_int4: M must be non-negative");
  // activation rows are addressed with 32-bit element offsets (grouped: a.M
  // slots bound every row the tile list or the row map can name)
  PF_CHECK((long)a.M * a.ldx < (1L << 31), "gemm_int4: activation offsets exceed 32 bits");
  const bool split = xk == XKind::SPLIT;
  if (tile_t == 64) {
    if (split) {
      if (grouped) dispatch_epi<64, true, true>(b, a, epi, prof_name);
      else dispatch_epi<64, true, false>(b, a, epi, prof_name);
    } else {
      if (grouped) dispatch_epi<64, false, true>(b, a, epi, prof_name);
      else dispatch_epi<64, false, false>(b, a, epi, prof_name);
    }
  } else {
    PF_CHECK(tile_t == 128, "gemm_int4: tile_t must be 64 or 128");
    if (split) {
      if (grouped) dispatch_epi<128, true, true>(b, a, epi, prof_name);
      else dispatch_epi<128, true, false>(b, a, epi, prof_name);
    } else {
      if (grouped) dispatch_epi<128, false, true>(b, a, epi, prof_name);
      else dispatch_epi<128, false, false>(b, a, epi, prof_name);
    }
  }
}

// ---------------------------------------------------------------- layout probe

__global__ void k_probe_mfma(const uint16_t* A, const uint16_t* B, float* D) {
  // A: 16x32 row-major fp16, B: 32x16 row-major fp16, D: 16x16 row-major f32
  const int l = threadIdx.x, l16 = l & 15, lg = l >> 4;
  h8_t a, bb;
  for (int i = 0; i < 8; ++i) {
    a[i] = __builtin_bit_cast(_Float16, A[l16 * 32 + 8 * lg + i]);
    bb[i] = __builtin_bit_cast(_Float16, B[(8 * lg + i) * 16 + l16]);
  }
  f4_t d = mfma16x16x32(a, bb, f4_t{0.f, 0.f, 0.f, 0.f});
  for (int r = 0; r < 4; ++r) D[(4 * lg + r) * 16 + l16] = d[r];
}

void probe_mfma_f16(pfhip_backend* b, const uint16_t* a, const uint16_t* bm, float* d) {
  ProfScope ps(b, "probe_mfma_f16");
  hipLaunchKernelGGL(k_probe_mfma, dim3(1), dim3(64), 0, b->stream, a, bm, d);
  PF_HIP(hipGetLastError());
}

}  // namespace pf
