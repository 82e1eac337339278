// gemm_w4.hip — MatMulNBits int4 GEMM with the block scale folded into the
// fp16 weights (the model forward's fast path).
//
// Computes out[t][n] = sum_k x[t][k] * w16[n][k] + bias[n] with
// w16[n][k] = fp16((q[n][k] - zp[n][b]) * scale[n][b]) — MatMulNBits
// (packages/textsift/src/zig/wasm_exports.zig:560-707) with the per-block
// scale applied to each weight in fp16 instead of to each block's partial
// sum in f32. The GPU paths of the reference feed these GEMMs fp16
// activations (src/native/backend.ts:557-576); the weight rounding adds an
// error of the same size as that activation rounding (2^-12 relative per
// product).
//
// Mapping to CDNA4:
//  * No weight staging through LDS and no per-block f32 scale update. Each
//    wave owns WF x 16 weight rows of the tile and reads its MFMA A-operand
//    fragments straight from HBM: lane (l16, lg) loads 16 bytes = one whole
//    quant block (32 nibbles) of row l16 at K offset 32*lg of the current
//    128-wide K chunk, and dequantises it in registers.
//  * K is permuted inside each 128-wide chunk: MFMA step j (0..3) takes the
//    8 values K = 32*lg + 8*j .. +7 from lane group lg. The activation
//    operand uses the same permutation, so the dot product is unchanged.
//  * Weights are repacked once (w4_repack): byte b of each dword holds k = b
//    in its low nibble and k = b + 4 in its high nibble. Two masks (no
//    shift) isolate the low and the high nibbles in their bytes, and one
//    v_perm_b32 per pair places two of them under exponent bytes: 0x64 for
//    the low nibbles ((1024 + q) as packed fp16), 0x54 for the high ones
//    ((64 + q): the nibble sits at mantissa bit 4, which weighs 1 at that
//    exponent), in natural k order. One packed add subtracts (1024 + zp) or
//    (64 + zp) exactly and one packed multiply applies the scale (the only
//    rounding).
//  * Activations are the shared operand: the workgroup's BT x 128 chunk is
//    copied HBM -> LDS with global_load_lds_dwordx4 (no register staging),
//    double buffered, in 256-byte rows whose 16-byte units are XOR-swizzled
//    by (row & 15) so the MFMA B-fragment reads (ds_read_b128) are
//    conflict-free.
//  * The GEMM is computed transposed (D = W . X^T) as in gemm_int4.hip, so
//    each lane ends with 4 consecutive output columns of one token and the
//    RoPE / SwiGLU epilogues are lane-local.
#include <type_traits>

#include "common.h"
#include "epilogue.h"
#include "pfhip_internal.h"
#include "topk.h"

namespace pf {

namespace {

constexpr int KC = 128;  // K per chunk (4 quant blocks, 256 bytes of fp16 activations per row)
constexpr int NW = 4;    // waves per workgroup, stacked along N

__device__ __forceinline__ uint32_t h2_bits(h2_t v) { return __builtin_bit_cast(uint32_t, v); }

// {cos, sin} of pairs pidx and pidx + 1 (pidx even) from row `row` of the
// LDS-staged RoPE table (128-byte rows, units swizzled by row & 7).
__device__ __forceinline__ h4_t rope_entry(const _Float16* tb, int row, int pidx) {
  const char* trow = reinterpret_cast<const char*>(tb) + row * 128;
  return *reinterpret_cast<const h4_t*>(trow + (((pidx >> 2) ^ (row & 7)) << 4) + (pidx & 3) * 4);
}

// One repacked dword (8 nibbles) -> fp16 (q - zp) * scale for k = 0..7.
// off = (-(1024 + zp), -(1024 + zp)), sc = (scale, scale).
// The low nibbles are masked into the low bits of each byte and placed under
// 0x64 exponent bytes: fp16 1024 + q (mantissa ulp 1). The high nibbles are
// masked in place (q << 4 in each byte, no shift) and placed under 0x54
// exponent bytes: fp16 64 + q (exponent 21: mantissa bit 4 weighs 2^6 * 16 /
// 1024 = 1). Their offset is -(64 + zp) = off + 960, exact like off. Both
// subtractions and the scale multiply give exactly the values of the
// single-magic form, with one shift fewer per dword.
__device__ __forceinline__ h2_t off_high(h2_t off) { return off + h2_t{(_Float16)960.0f, (_Float16)960.0f}; }
__device__ __forceinline__ h8_t dequant_fold(uint32_t w, h2_t off, h2_t off_hi, h2_t sc) {
  const uint32_t lo = w & 0x0F0F0F0Fu;          // k0 k1 k2 k3 (one per byte, bits 0-3)
  const uint32_t hi = w & 0xF0F0F0F0u;          // k4 k5 k6 k7 (one per byte, bits 4-7)
  const uint32_t M = 0x64646464u;               // exponent bytes of 1024
  const uint32_t MH = 0x54545454u;              // exponent bytes of 64
  const uint32_t p0 = __builtin_amdgcn_perm(M, lo, 0x04010400u);   // (1024 + k0, 1024 + k1)
  const uint32_t p1 = __builtin_amdgcn_perm(M, lo, 0x04030402u);
  const uint32_t p2 = __builtin_amdgcn_perm(MH, hi, 0x04010400u);  // (64 + k4, 64 + k5)
  const uint32_t p3 = __builtin_amdgcn_perm(MH, hi, 0x04030402u);
  const h2_t d0 = (__builtin_bit_cast(h2_t, p0) + off) * sc;
  const h2_t d1 = (__builtin_bit_cast(h2_t, p1) + off) * sc;
  const h2_t d2 = (__builtin_bit_cast(h2_t, p2) + off_hi) * sc;
  const h2_t d3 = (__builtin_bit_cast(h2_t, p3) + off_hi) * sc;
  return __builtin_bit_cast(h8_t, u4_t{h2_bits(d0), h2_bits(d1), h2_bits(d2), h2_bits(d3)});
}

__device__ __forceinline__ int xcd_remap(int bid, int total) {
  const int xcd = bid & 7, idx = bid >> 3;
  const int per = total >> 3, rem = total & 7;
  return xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
}

// Geometry of the LDS-staged output of a (WF, BT) tile: ESZ output bytes per
// element, CF output columns per 16-row fragment, FB bytes per row of one
// fragment, PS bytes one lane holds per fragment row; the tile is staged in
// NP passes of FG fragments per wave (PRB bytes per staged row, UP 16-byte
// units, units XOR-swizzled by row & SWM for conflict-free LDS writes).
template <int WF, int BT, Epi EPI, int NW = 4>
struct StagedOut {
  static constexpr bool F32OUT = EPI == Epi::F32 || EPI == Epi::F32_TOPK;
  static constexpr int ESZ = F32OUT ? 4 : 2;
  static constexpr int CF = EPI == Epi::SWIGLU_F16 ? 8 : 16;
  static constexpr int FB = CF * ESZ;
  static constexpr int PS = FB / 4;
  static constexpr int NP = (NW * WF * FB * BT > 65536 && WF % 2 == 0) ? 2 : 1;
  static constexpr int FG = WF / NP;
  static constexpr int PRB = NW * FG * FB;
  static constexpr int UP = PRB / 16;
  static constexpr int SWM = UP % 16 == 0 ? 15 : (UP % 8 == 0 ? 7 : (UP % 4 == 0 ? 3 : 0));
  static constexpr size_t LDS = (size_t)BT * PRB;
  // (small tiles store directly: fewer units than threads)
  static constexpr bool OK = (F32OUT || EPI == Epi::F16 || EPI == Epi::ROPE_F16 || EPI == Epi::SWIGLU_F16) &&
                             BT * UP % (64 * NW) == 0;
};

// NW waves per workgroup (4: two workgroups per CU; 8 measured on a
// 256-token tile: each dequantised fragment feeds twice the MFMAs, but the
// doubled activation reads from LDS cancel it: gate_up -2 %, down +10 %)
// CT > 0 (small tiles): K / 128 at compile time; every chunk's activations
// and weights are loaded at once, so a workgroup waits for memory once
// instead of once per chunk (the latency that dominates when a GEMM is a few
// workgroups).
// EVENC (CT == 0 only): K / 128 is even. The chunk loop is unrolled by two
// with the last chunk's register set fixed at compile time (a run-time choice
// between the two sets made the 128-row tiles spill).
// W16: the weights are fp16 [N][K] (p.w16; no quantisation, no dequantisation):
// BASELINE config 3's fp16 router (the 64- and 128-row tiles, and the all-K
// 16-row tile, whose 5 chunks of fp16 weights take 160 registers).
struct W16Reg {
  u4_t v[4];
};
template <int WF, int BT, int XS, Epi EPI, bool GROUPED, int NW = 4, int CT = 0, bool NORM = false,
          bool EVENC = false, bool W16 = false>
__global__ __launch_bounds__(64 * NW, 8 / NW) void k_gemm_w4(GemmArgs p) {
  static_assert(!W16 || !GROUPED, "fp16 weights: dense tiles only");
  constexpr int BN = NW * WF * 16;  // weight rows per workgroup
  constexpr int TJ = BT / 16;       // token fragments per wave
  constexpr int XI = BT / (4 * NW);  // 1 KB (4-row) direct loads per wave per plane per chunk
  static_assert(XI >= 1 && BT % (4 * NW) == 0, "whole 4-row copies per wave");
  constexpr int PLANE = BT * KC;    // halves per plane per buffer

  extern __shared__ __attribute__((aligned(16))) _Float16 xs_lds[];  // [2][XS][BT][KC] swizzled

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;

  const int n_tiles = (p.N + BN - 1) / BN;
  // Grouped: the grid covers the largest possible tile list; only the first
  // num_tiles x n_tiles workgroups have work. Those are spread round-robin
  // over the XCDs by the hardware, and the XCD remap is taken over them alone
  // (over the whole grid it would put all the work on the first XCDs).
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
  // Weight fragments per wave: WF, or WF / 2 when the rows from n0 to N fit
  // in half the tile (the last tile of an N that is not a multiple of BN:
  // down's 640 = 2.5 x 256, QKV's 1152 = 4.5 x 256). Fragment f of wave w
  // holds rows n0 + (w nf + f) 16 .. + 15, so a half tile spreads its rows
  // over every wave and takes half the time. A wave whose rows all lie past
  // N loads no weights and issues no dequantisation or MFMAs; it still
  // copies its share of the activations and joins every barrier. Both are
  // wave-uniform. (The all-K tiles, CT > 0, keep every wave busy: guarding
  // their loads spills.)
  constexpr bool HALF = CT == 0 && WF % 2 == 0 && !W16 && StagedOut<WF, BT, EPI, NW>::NP == 1 &&
                        EPI == Epi::F16 && GROUPED;
  const bool half = HALF && p.N - n0 <= NW * (WF / 2) * 16;
  const int nf = half ? WF / 2 : WF;
  const bool idle = CT == 0 && n0 + wave * nf * 16 >= p.N;
  const int K = p.K;
  const int C = K / KC;
  const int kd = K >> 3;   // dwords per packed weight row
  const int nb = K >> 5;   // quant blocks per row

  // ---- weight fragments: buffer loads from the expert's weights and
  // scale pairs (one descriptor each, in scalar registers) at fixed per-lane
  // byte offsets, the chunk in the scalar offset: no address arithmetic per
  // load (rows past N read row N-1; never stored). The host checks that the
  // matrices' byte sizes fit the descriptors' 31-bit range.
  const __amdgpu_buffer_rsrc_t wrs =
      W16 ? __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.w16), 0, p.N * K * 2, 0x00020000)
          : __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p.w + (size_t)expert * p.w_gs), 0, p.N * kd * 4,
                                              0x00020000);
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(p.wsz + (size_t)expert * p.wsz_gs), 0, p.N * nb * 4, 0x00020000);
  uint32_t woff[WF], soff[WF];
#pragma unroll
  for (int f = 0; f < WF; ++f) {
    const int n = min(n0 + (wave * nf + f) * 16 + l16, p.N - 1);
    woff[f] = W16 ? (uint32_t)(n * K + lg * 32) * 2u : (uint32_t)(n * kd + lg * 4) * 4u;
    soff[f] = (uint32_t)(n * nb + lg) * 4u;
  }

  // ---- chunk 0's weights and the bias are issued here: their addresses
  // need only the tile entry, so their latency overlaps the reads of the
  // activation rows' indices (row_map) below.
  using WR = std::conditional_t<W16, W16Reg, u4_t>;
  WR wraw[WF], wnext[WF];
  uint32_t sz[WF], sznext[WF];
  // (nfc: std::integral_constant, the fragments loaded: WF, or WF / 2 in a half tile)
  auto load_w = [&](auto nfc, int c, WR* wr, uint32_t* s) {
#pragma unroll
    for (int f = 0; f < decltype(nfc)::value; ++f) {
      if constexpr (W16) {
        // chunk c: this lane's 32 consecutive values (64 bytes), one 16-byte unit per MFMA step
#pragma unroll
        for (int j = 0; j < 4; ++j) wr[f].v[j] = __builtin_amdgcn_raw_buffer_load_b128(wrs, woff[f], c * 256 + j * 16, 0);
        s[f] = 0u;
      } else {
        // chunk c: 128 values = 64 bytes of each row, and its 4 quant blocks' pairs
        wr[f] = __builtin_amdgcn_raw_buffer_load_b128(wrs, woff[f], c * 64, 0);
        s[f] = __builtin_amdgcn_raw_buffer_load_b32(srs, soff[f], c * 16, 0);
      }
    }
  };

  // The accumulators start at the bias of the lane's 4 columns of each
  // fragment (the MFMAs add onto it); columns past N get 0 and are never
  // stored. Loads are unconditional (indices clamped). The bias widens with
  // the hardware conversion (this GEMM serves the fp16 numerics, the GPU
  // shaders' arithmetic).
  const uint16_t* __restrict__ BIAS = p.bias ? p.bias + (size_t)expert * p.bias_gs : nullptr;
  int ncol[WF];
#pragma unroll
  for (int f = 0; f < WF; ++f) ncol[f] = n0 + (wave * nf + f) * 16 + 4 * lg;
  u2_t braw[WF];
#pragma unroll
  for (int f = 0; f < WF; ++f) braw[f] = u2_t{0u, 0u};
  if (BIAS) {
    if ((p.N & 3) == 0 && (reinterpret_cast<uintptr_t>(BIAS) & 7) == 0) {
#pragma unroll
      for (int f = 0; f < WF; ++f) braw[f] = *reinterpret_cast<const u2_t*>(BIAS + min(ncol[f], p.N - 4));
    } else {
#pragma unroll
      for (int f = 0; f < WF; ++f) {
        uint32_t h[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) h[r] = BIAS[min(ncol[f] + r, p.N - 1)];
        braw[f] = u2_t{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
      }
    }
  }
  // (the K-looped tiles call it once the first chunk's loads are issued:
  // waiting for the bias then overlaps their latency instead of preceding them)
  f4_t acc[WF][TJ];
  auto init_acc = [&]() {
#pragma unroll
    for (int f = 0; f < WF; ++f) {
      const uint32_t bw[2] = {braw[f].x, braw[f].y};
      float bv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r)
        bv[r] = ncol[f] + r < p.N ? (float)__builtin_bit_cast(_Float16, (uint16_t)(bw[r >> 1] >> (16 * (r & 1))))
                                  : 0.0f;
#pragma unroll
      for (int j = 0; j < TJ; ++j) acc[f][j] = f4_t{bv[0], bv[1], bv[2], bv[3]};
    }
  };
  // (not in the kernels with half tiles: the two register sets then held
  // across the row indices' reads spill)
  if constexpr (CT == 0 && !HALF)
    if (!idle) load_w(std::integral_constant<int, WF>{}, 0, wraw, sz);

  // ---- activation rows this lane copies (rows past the tile read the
  // tile's last row; their outputs are never stored)
  const uint16_t* __restrict__ xsrc[XS];
  xsrc[0] = static_cast<const uint16_t*>(p.x);
  if constexpr (XS == 2) xsrc[1] = p.x_lo;
  int xoff[XI];
#pragma unroll
  for (int m = 0; m < XI; ++m) {
    const int r = (m * NW + wave) * 4 + lg;
    const int lr = row0 + min(r, rows - 1);
    const int g = p.row_map ? p.row_map[lr] : lr;
    xoff[m] = g * p.ldx + ((l16 ^ (r & 15)) << 3);
  }

  // (byte offsets as unsigned 32-bit values from a uniform base: the loads
  // take the scalar-base + 32-bit-offset form, no 64-bit address arithmetic)
  auto load_x = [&](int c, int buf) {
#pragma unroll
    for (int pl = 0; pl < XS; ++pl)
#pragma unroll
      for (int m = 0; m < XI; ++m) {
        _Float16* dst = xs_lds + (buf * XS + pl) * PLANE + (m * NW + wave) * 512;
        copy16_to_lds(reinterpret_cast<const char*>(xsrc[pl]) + (uint32_t)(xoff[m] + c * KC) * 2u, (lds_ptr_t)dst);
      }
  };

  // one 128-wide K chunk of MFMAs from LDS buffer buf and the weights in wraw / sz
  // (fragments 0 .. nfc - 1)
  auto compute = [&](auto nfc, int buf, const WR (&wr)[WF], const uint32_t (&szc)[WF]) {
    constexpr int NF = decltype(nfc)::value;
    h2_t off[WF], offh[WF], sc[WF];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const h2_t pr = __builtin_bit_cast(h2_t, szc[f]);
      off[f] = h2_t{pr.x, pr.x};
      offh[f] = off_high(off[f]);
      sc[f] = h2_t{pr.y, pr.y};
    }
    const _Float16* xb = xs_lds + buf * XS * PLANE;
    if constexpr (TJ == 1 && XS == 1) {
      // one token fragment (the 16-row tiles): the chunk's four activation
      // fragments are read before its MFMAs, so the LDS latency is paid once
      // per chunk instead of once per step (the steps are otherwise a serial
      // chain of LDS read, wait, MFMA)
      h8_t xh[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) xh[j] = *reinterpret_cast<const h8_t*>(xb + l16 * KC + (((4 * lg + j) ^ l16) << 3));
      __builtin_amdgcn_sched_barrier(0);  // (the scheduler would sink the reads next to their MFMAs)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int f = 0; f < NF; ++f) {
          h8_t wd;
          if constexpr (W16) wd = __builtin_bit_cast(h8_t, wr[f].v[j]);
          else wd = dequant_fold(wr[f][j], off[f], offh[f], sc[f]);
          acc[f][0] = mfma16x16x32(wd, xh[j], acc[f][0]);
        }
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      h8_t wd[WF];
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        if constexpr (W16) wd[f] = __builtin_bit_cast(h8_t, wr[f].v[j]);
        else wd[f] = dequant_fold(wr[f][j], off[f], offh[f], sc[f]);
      }
      const int unit = ((4 * lg + j) ^ l16) << 3;
      if constexpr (XS == 1) {
        // token fragment tj + 1's activations are read before fragment tj's
        // MFMAs, pinned there by the scheduling barrier (the scheduler would
        // sink each read next to its MFMAs and wait out the LDS latency once
        // per fragment): gate_up -3 %, QKV -5 %
        h8_t xa = *reinterpret_cast<const h8_t*>(xb + l16 * KC + unit);
#pragma unroll
        for (int tj = 0; tj < TJ; ++tj) {
          h8_t xn = xa;
          if (tj + 1 < TJ) xn = *reinterpret_cast<const h8_t*>(xb + (16 * (tj + 1) + l16) * KC + unit);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int f = 0; f < NF; ++f) acc[f][tj] = mfma16x16x32(wd[f], xa, acc[f][tj]);
          xa = xn;
        }
      } else {
#pragma unroll
        for (int tj = 0; tj < TJ; ++tj) {
          const int o = (16 * tj + l16) * KC + unit;
          const h8_t xh = *reinterpret_cast<const h8_t*>(xb + o);
          const h8_t xl = *reinterpret_cast<const h8_t*>(xb + PLANE + o);
#pragma unroll
          for (int f = 0; f < NF; ++f) acc[f][tj] = mfma16x16x32(wd[f], xh, acc[f][tj]);
#pragma unroll
          for (int f = 0; f < NF; ++f) acc[f][tj] = mfma16x16x32(wd[f], xl, acc[f][tj]);
        }
      }
    }
  };

  [[maybe_unused]] WR wall[CT > 0 ? CT : 1][WF];
  [[maybe_unused]] uint32_t szall[CT > 0 ? CT : 1][WF];
  if constexpr (CT > 0) {
    // (the all-K tiles widen the bias before their loads: after them it
    // costs a spilled register and gains nothing at their sizes)
    init_acc();
#pragma unroll
    for (int c = 0; c < CT; ++c) {
      load_x(c, c);
      load_w(std::integral_constant<int, WF>{}, c, wall[c], szall[c]);
    }
    [[maybe_unused]] u4_t gam[CT];
    if constexpr (NORM) {
      // the residual rows into buffers CT .. 2 CT - 1, in the same layout
#pragma unroll
      for (int c = 0; c < CT; ++c)
#pragma unroll
        for (int m = 0; m < XI; ++m)
          copy16_to_lds(p.nrm_res + xoff[m] + c * KC, (lds_ptr_t)(xs_lds + (CT + c) * PLANE + (m * NW + wave) * 512));
      // and this thread's gamma units (see below), under the same wait
      const int q = tid & 15;
#pragma unroll
      for (int f = 0; f < CT; ++f)
        gam[f] = *reinterpret_cast<const u4_t*>(p.nrm_gamma + (5 * (q >> 1) + f) * 16 + 8 * (q & 1));
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if constexpr (NORM) {
      // 16 threads per row: h2 = fp16(o + res), the row's sum of squares of
      // the f32 sums, xn = fp16(h2 inv_rms gamma) stored to memory and over o
      // for the MFMAs. The sum of squares is taken in exactly the order of
      // the fused O kernel's epilogue (k_gemm_w4_rownorm below), so both
      // forms give bit-identical h2 and xn and a sequence's result does not
      // depend on the batch size that selects the form: there, lane group lg
      // of wave w sums fma(s, s, .) over columns (5 w + f) 16 + 4 lg + 0..3
      // for f = 0..4 in that order, lane groups combine as (P0 + P1) +
      // (P2 + P3) and the 8 wave sums are added in order. Here thread
      // q = 2 w + h holds the 16-byte unit at column (5 w + f) 16 + 8 h of
      // every f, i.e. the columns of lane groups 2 h and 2 h + 1.
      static_assert(BT * 16 == 64 * NW && XS == 1 && CT == 5, "row normalisation: 16 threads per 640-wide row");
      const int r = tid >> 4, q = tid & 15;
      const int w8 = q >> 1, hh = q & 1;
      u4_t hs[CT];
      int slot[CT], colf[CT];
      float pa = 0.0f, pb = 0.0f;
#pragma unroll
      for (int f = 0; f < CT; ++f) {
        colf[f] = (5 * w8 + f) * 16 + 8 * hh;
        slot[f] = (colf[f] >> 7) * PLANE + r * KC + ((((colf[f] & 127) >> 3) ^ (r & 15)) << 3);
        const h8_t o8 = *reinterpret_cast<const h8_t*>(xs_lds + slot[f]);
        const h8_t r8 = *reinterpret_cast<const h8_t*>(xs_lds + CT * PLANE + slot[f]);
        float sv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) sv[i] = (float)o8[i] + (float)r8[i];
#pragma unroll
        for (int i = 0; i < 4; ++i) pa = fmaf(sv[i], sv[i], pa);
#pragma unroll
        for (int i = 4; i < 8; ++i) pb = fmaf(sv[i], sv[i], pb);
        const u2_t lo = to_f16x4_native(sv), hi = to_f16x4_native(sv + 4);
        hs[f] = u4_t{lo.x, lo.y, hi.x, hi.y};
      }
      float qv = pa + pb;
      qv += __shfl_xor(qv, 1, 64);
      float tot = 0.0f;
#pragma unroll
      for (int w = 0; w < 8; ++w) tot += __shfl(qv, (lane & ~15) + 2 * w, 64);
      const float inv_rms = 1.0f / sqrtf(tot * (1.0f / (float)(CT * KC)) + p.nrm_eps);
      const bool store = r < rows;
      const size_t orow = (size_t)(row0 + r) * (CT * KC);
      __syncthreads();  // every thread has read its o and residual units
#pragma unroll
      for (int f = 0; f < CT; ++f) {
        const h8_t h8 = __builtin_bit_cast(h8_t, hs[f]);
        const h8_t g8 = __builtin_bit_cast(h8_t, gam[f]);
        float y[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = (float)h8[i] * inv_rms * (float)g8[i];
        const u2_t lo = to_f16x4_native(y), hi = to_f16x4_native(y + 4);
        const u4_t xv = u4_t{lo.x, lo.y, hi.x, hi.y};
        *reinterpret_cast<u4_t*>(xs_lds + slot[f]) = xv;
        if (store) {
          *reinterpret_cast<u4_t*>(p.nrm_h + orow + colf[f]) = hs[f];
          *reinterpret_cast<u4_t*>(p.nrm_xn + orow + colf[f]) = xv;
        }
      }
      __syncthreads();
    }
  } else {
    // chunk c's weights are in register set A (wraw, sz) for even c and B
    // (wnext, sznext) for odd c, its activations in LDS buffer c & 1: the
    // loop is unrolled by two so that neither the register sets nor the
    // buffer addresses change at run time (no register copies per chunk)
    // (a half tile runs its own copy of the loop, over WF / 2 fragments)
    auto kloop = [&](auto nfc) {
      auto step = [&](int c, int buf, const WR (&wc)[WF], const uint32_t (&scc)[WF], WR (&wn)[WF],
                      uint32_t (&sn)[WF]) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        load_x(c + 1, buf ^ 1);
        if (!idle) load_w(nfc, c + 1, wn, sn);
        // the expert GEMMs raise the wave's issue priority over the chunk's
        // MFMAs and dequantisation (and drop it for the loads and the barrier):
        // gate_up 235 -> 229 us, down -1 us; the dense QKV GEMM got slower with it
        if constexpr (GROUPED) __builtin_amdgcn_s_setprio(1);
        if (!idle) compute(nfc, buf, wc, scc);
        if constexpr (GROUPED) __builtin_amdgcn_s_setprio(0);
      };
      load_x(0, 0);
      if constexpr (HALF)
        if (!idle) load_w(nfc, 0, wraw, sz);
      init_acc();
      int c = 0;
      for (; c + 2 < C; c += 2) {
        step(c, 0, wraw, sz, wnext, sznext);
        step(c + 1, 1, wnext, sznext, wraw, sz);
      }
      if constexpr (EVENC) step(c, 0, wraw, sz, wnext, sznext);  // the last chunk, C - 1, is then in set B
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    };
    if (half) kloop(std::integral_constant<int, HALF ? WF / 2 : WF>{});
    else kloop(std::integral_constant<int, WF>{});
  }

  // ---- RoPE operands, loaded before the last chunk's MFMAs so that their
  // latency overlaps them.
  // RoPE: the table rows (32 (cos, sin) fp16 pairs = 128 bytes) of the
  // tile's BT positions are copied into the LDS buffer the last chunk does
  // not use, their eight 16-byte units XOR-swizzled by (row & 7). Row r of
  // the tile is at position (row0 + r) mod seq_len. One wave instruction
  // fills 8 rows.
  // (with CT > 0 every chunk buffer is in use and the table goes after them)
  const int tbuf = CT > 0 ? CT : (C & 1);
  if constexpr (EPI == Epi::ROPE_F16) {
    static_assert(BT % 8 == 0, "RoPE table staging: whole 8-row copies");
    const int p0 = (int)((uint32_t)row0 % (uint32_t)p.seq_len);
    _Float16* tb = xs_lds + tbuf * XS * PLANE;
    for (int u8 = wave; u8 < BT / 8; u8 += NW) {  // wave-uniform
      const int r = u8 * 8 + (lane >> 3);
      int q = p0 + r;
      if (p.seq_len >= BT) q = q >= p.seq_len ? q - p.seq_len : q;
      else q %= p.seq_len;
      const int u = (lane & 7) ^ (r & 7);  // this lane's unit lands at position lane & 7 of row r
      copy16_to_lds(p.rope_pairs + (size_t)q * 64 + u * 8, (lds_ptr_t)(tb + u8 * 512));
    }
  }

  if constexpr (CT > 0) {
#pragma unroll
    for (int c = 0; c < CT; ++c) compute(std::integral_constant<int, WF>{}, c, wall[c], szall[c]);
  } else if (!idle) {
    auto last = [&](auto nfc) {
      if constexpr (EVENC) compute(nfc, 1, wnext, sznext);
      else compute(nfc, 0, wraw, sz);
    };
    if (half) last(std::integral_constant<int, HALF ? WF / 2 : WF>{});
    else last(std::integral_constant<int, WF>{});
  }
  // the SwiGLU epilogue's clamp reads the accumulators with inline assembly
  if constexpr (EPI == Epi::SWIGLU_F16) {
#pragma unroll
    for (int f = 0; f < WF; ++f) mfma_settled(acc[f]);
  }
  if constexpr (EPI == Epi::ROPE_F16) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  // ---- epilogue: lane holds out[token = 16 tj + l16][n = n0 + (wave WF + f) 16 + 4 lg + r]
  using SO = StagedOut<WF, BT, EPI, NW>;
  if (SO::OK && p.out_staged) {
    // The tile goes out through LDS: lanes write their values in row-major
    // order, then every lane stores whole 16-byte units of consecutive
    // columns, so each row segment of the tile leaves as full lines (the
    // direct form writes 4- to 16-byte pieces of 16 rows per instruction,
    // which costs the gate_up GEMM about a fifth of its time).
    char* ob = reinterpret_cast<char*>(xs_lds);
    u2_t ow[WF][TJ];  // packed fp16 results (F32 writes the accumulators)
    if constexpr (!SO::F32OUT) {
#pragma unroll
      for (int f = 0; f < WF; ++f) {
        const bool rope = EPI == Epi::ROPE_F16 && n0 + (wave * nf + f) * 16 < p.rope_cols;
        const int pidx = (ncol[f] & 63) >> 1;
#pragma unroll
        for (int tj = 0; tj < TJ; ++tj) {
          const float v[4] = {acc[f][tj][0], acc[f][tj][1], acc[f][tj][2], acc[f][tj][3]};
          if constexpr (EPI == Epi::ROPE_F16) {
            if (rope) {
              const int row = 16 * tj + l16;
              ow[f][tj] = rope_f16x4_native(v, rope_entry(xs_lds + tbuf * XS * PLANE, row, pidx));
            } else {
              ow[f][tj] = to_f16x4_native(v);
            }
          } else if constexpr (EPI == Epi::F16) {
            ow[f][tj] = to_f16x4_native(v);
          } else {
            ow[f][tj] = u2_t{swiglu_f16x2_native<true>(v), 0u};
          }
        }
      }
    }
    // top-k epilogue: the tile's rows per expert, in LDS after the staged
    // tile (inside the activation buffers, free now), cleared here
    [[maybe_unused]] int* topk_hist = reinterpret_cast<int*>(ob + SO::LDS);
#pragma unroll
    for (int ps = 0; ps < SO::NP; ++ps) {
      __syncthreads();  // every wave is done with the LDS buffers (and the previous pass)
      if constexpr (EPI == Epi::F32_TOPK)
        if (ps == 0 && p.topk_counts && tid < 128) topk_hist[tid] = 0;
#pragma unroll
      for (int fl = 0; fl < SO::FG; ++fl) {
        const int f = ps * SO::FG + fl;
#pragma unroll
        for (int tj = 0; tj < TJ; ++tj) {
          const int row = 16 * tj + l16;
          // (one pass in the kernels with half tiles: fragment wave nf + f at
          // its column position; past the half tile's fragments nothing is
          // staged and the stores below skip those columns, all past N)
          if (HALF && f >= nf) continue;
          const int byte = (HALF ? (wave * nf + f) * SO::FB : (wave * SO::FG + fl) * SO::FB) + lg * SO::PS;
          char* dst = ob + row * SO::PRB + (((byte >> 4) ^ (row & SO::SWM)) << 4) + (byte & 15);
          if constexpr (SO::F32OUT) *reinterpret_cast<f4_t*>(dst) = acc[f][tj];
          else if constexpr (EPI == Epi::SWIGLU_F16) *reinterpret_cast<uint32_t*>(dst) = ow[f][tj].x;
          else *reinterpret_cast<u2_t*>(dst) = ow[f][tj];
        }
      }
      __syncthreads();
      const int ocol0 = EPI == Epi::SWIGLU_F16 ? n0 / 2 : n0;
      const int oN = EPI == Epi::SWIGLU_F16 ? p.N / 2 : p.N;
#pragma unroll
      for (int i = 0; i < BT * SO::UP / (64 * NW); ++i) {
        const int idx = i * (64 * NW) + tid, row = idx / SO::UP, up = idx % SO::UP;
        const int byte = ((up ^ (row & SO::SWM)) << 4);
        const int w = byte / (SO::FG * SO::FB), within = byte % (SO::FG * SO::FB);
        const int col = ocol0 + (w * WF + ps * SO::FG) * SO::CF + within / SO::ESZ;
        // (the top-k epilogue may be given no logits output: it reads them from LDS)
        if (row < rows && col < oN && (EPI != Epi::F32_TOPK || p.out)) {
          u4_t* dstp =
              reinterpret_cast<u4_t*>(static_cast<char*>(p.out) + ((size_t)(row0 + row) * p.ldo + col) * SO::ESZ);
          const u4_t val = *reinterpret_cast<const u4_t*>(ob + row * SO::PRB + (up << 4));
          // the expert outputs (grouped fp16: the down GEMM) are read once,
          // by the combine: non-temporal stores (down 150 -> 144 us)
          if constexpr (GROUPED && EPI == Epi::F16) __builtin_nontemporal_store(val, dstp);
          else *dstp = val;
        }
      }
    }
    if constexpr (EPI == Epi::F32_TOPK && SO::NP == 1 && BN == 128) {
      // Router top-4 of every row from the staged tile (all N == 128 logits
      // of BT rows are in LDS). TPR threads share a row, each taking the
      // top-4 of SEG consecutive logits by the reference's insertion rule;
      // the lists then merge pairwise by (value descending, index
      // ascending), the lower segment winning ties, which is what the
      // insertion over the whole row yields without NaNs. A row with a NaN
      // replays the sequential insertion over all 128 logits.
      constexpr int TPR = 64 * NW / BT, SEG = 128 / TPR;
      static_assert(TPR >= 2 && TPR <= 32 && (TPR & (TPR - 1)) == 0, "top-k: 2..32 threads per row");
      const int row = tid / TPR, part = tid % TPR;
      const char* rb = ob + row * SO::PRB;
      auto at = [&](int c) -> float {
        return *reinterpret_cast<const float*>(rb + (((c >> 2) ^ (row & SO::SWM)) << 4) + (c & 3) * 4);
      };
      bool nan = false;
#pragma unroll
      for (int u = 0; u < SEG / 4; ++u) {
        const f4_t q = *reinterpret_cast<const f4_t*>(rb + ((((SEG / 4) * part + u) ^ (row & SO::SWM)) << 4));
        nan = nan | (q[0] != q[0]) | (q[1] != q[1]) | (q[2] != q[2]) | (q[3] != q[3]);
      }
      float V[4];
      int I[4];
      if constexpr (SEG == 8) {
        // short segments: branch-free selection on (value, index) keys;
        // a row with a NaN takes the sequential path below
        uint64_t ka[4], kb[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          ka[c] = topk_key(at(SEG * part + c), SEG * part + c);
          kb[c] = topk_key(at(SEG * part + 4 + c), SEG * part + 4 + c);
        }
        topk_sort4(ka);
        topk_sort4(kb);
        topk_merge4(ka, kb);
#pragma unroll
        for (int sft = 1; sft < TPR; sft <<= 1) {
          nan = nan | (__shfl_xor((int)nan, sft, 64) != 0);
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const uint32_t lo = __shfl_xor((uint32_t)ka[k], sft, 64);
            const uint32_t hi = __shfl_xor((uint32_t)(ka[k] >> 32), sft, 64);
            kb[k] = ((uint64_t)hi << 32) | lo;
          }
          topk_merge4(ka, kb);  // keys are distinct: both threads of a pair get the same list
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          I[k] = topk_key_index(ka[k]);
          V[k] = at(I[k]);
        }
      } else {
      topk_insertion<4>([&](int c) { return at(SEG * part + c); }, SEG, V, I);
#pragma unroll
      for (int k = 0; k < 4; ++k) I[k] += SEG * part;
#pragma unroll
      for (int sft = 1; sft < TPR; sft <<= 1) {
        nan = nan | (__shfl_xor((int)nan, sft, 64) != 0);
        float OV[4];
        int OI[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          OV[k] = __shfl_xor(V[k], sft, 64);
          OI[k] = __shfl_xor(I[k], sft, 64);
        }
        // A: the lower segment's list, B: the upper one's
        const bool lower = (part & sft) == 0;
        float AV[4], BV[4], RV[4];
        int AI[4], BI[4], RI[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          AV[k] = lower ? V[k] : OV[k];
          AI[k] = lower ? I[k] : OI[k];
          BV[k] = lower ? OV[k] : V[k];
          BI[k] = lower ? OI[k] : I[k];
          RV[k] = 0.0f;
          RI[k] = 0;
        }
        // rank of each candidate among the 8
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          int ra = i, rbk = i;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            ra += BV[j] > AV[i];
            rbk += AV[j] >= BV[i];
          }
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            if (ra == k) {
              RV[k] = AV[i];
              RI[k] = AI[i];
            }
            if (rbk == k) {
              RV[k] = BV[i];
              RI[k] = BI[i];
            }
          }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          V[k] = RV[k];
          I[k] = RI[k];
        }
      }
      }
      // (the single-tile routing plan: each expert's bitmap of the tile's
      // rows, after the counters in LDS)
      [[maybe_unused]] uint32_t* pbits = reinterpret_cast<uint32_t*>(topk_hist + 128);
      if constexpr (BT == 16) {
        if (p.plan_slot_of) {  // (uniform)
          if (tid < 128) pbits[tid] = 0u;
          __syncthreads();
        }
      }
      if (part == 0 && row < rows) {
        if (nan) topk_insertion<4>(at, 128, V, I);
        const size_t t = (size_t)(row0 + row);
        topk_write<4>(V, I, p.topk_wscale, p.topk_idx + t * 4, p.topk_w + t * 4);
        if (p.topk_counts) {
#pragma unroll
          for (int k = 0; k < 4; ++k) atomicAdd(&topk_hist[I[k]], 1);  // order-free: the counts are exact
        }
        if constexpr (BT == 16) {
          if (p.plan_slot_of) {
#pragma unroll
            for (int k = 0; k < 4; ++k) atomicOr(&pbits[I[k]], 1u << row);  // order-free
          }
        }
      }
      if (p.topk_counts) {
        __syncthreads();
        if (tid < 128) p.topk_counts[(size_t)(row0 / BT) * 128 + tid] = topk_hist[tid];
      }
      if constexpr (BT == 16) {
        if (p.plan_slot_of) {
          // The routing plan of the tile's rows (M <= 16, one workgroup),
          // the outputs of moe_route's single-block kernel: expert e's rows
          // are its tokens in ascending order (bitmap ranks), experts in
          // ascending order, tiles of plan_tile_t rows.
          __syncthreads();
          int* poff = topk_hist + 256;  // [128] row offsets, [128] tile offsets, [4] wave sums
          int* ptoff = poff + 128;
          int* pws = ptoff + 128;
          int c = 0, ci = 0, ni = 0, n = 0;
          if (tid < 128) {
            c = __popc(pbits[tid]);
            n = (c + p.plan_tile_t - 1) / p.plan_tile_t;
            ci = c;
            ni = n;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
              const int a = __shfl_up(ci, o, 64), bb = __shfl_up(ni, o, 64);
              if (lane >= o) {
                ci += a;
                ni += bb;
              }
            }
            if (lane == 63) {
              pws[2 * wave] = ci;
              pws[2 * wave + 1] = ni;
            }
          }
          __syncthreads();
          const int total = pws[0] + pws[2], ntl = pws[1] + pws[3];
          if (tid < 128) {
            const int base = (wave == 1 ? pws[0] : 0) + ci - c;
            poff[tid] = base;
            ptoff[tid] = (wave == 1 ? pws[1] : 0) + ni - n;
            p.plan_expert_off[tid] = base;
          }
          if (tid == 0) {
            p.plan_expert_off[128] = total;
            *p.plan_num_tiles = ntl;
          }
          __syncthreads();
          for (int ti = tid; ti < ntl; ti += 64 * NW) {
            int lo = 0, hi = 127;
            while (lo < hi) {
              const int mid = (lo + hi + 1) >> 1;
              if (ptoff[mid] <= ti) lo = mid;
              else hi = mid - 1;
            }
            const int tot = (lo < 127 ? poff[lo + 1] : total) - poff[lo];
            const int r0 = (ti - ptoff[lo]) * p.plan_tile_t;
            reinterpret_cast<int4*>(p.plan_tiles)[ti] = int4{lo, poff[lo] + r0, min(p.plan_tile_t, tot - r0), 0};
          }
          if (part == 0 && row < rows) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              const int e = I[k];
              const int pos = poff[e] + __popc(pbits[e] & ((1u << row) - 1u));
              p.plan_slot_token[pos] = row0 + row;
              p.plan_slot_of[(size_t)(row0 + row) * 4 + k] = pos;
            }
          }
        }
      }
    }
    return;
  }

#pragma unroll
  for (int f = 0; f < WF; ++f) {
    const int n = ncol[f];
    if (f >= nf || n >= p.N) continue;
    // a fragment of 16 columns lies wholly below or above rope_cols (a multiple of 64)
    const bool rope = EPI == Epi::ROPE_F16 && n0 + (wave * nf + f) * 16 < p.rope_cols;
    const int pidx = (n & 63) >> 1;  // this lane's first (cos, sin) pair of the head
#pragma unroll
    for (int tj = 0; tj < TJ; ++tj) {
      const int lt = 16 * tj + l16;
      if (lt >= rows) continue;
      const size_t orow = (size_t)(row0 + lt);
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = acc[f][tj][r];
      if constexpr (EPI == Epi::ROPE_F16) {
        u2_t hv;
        if (rope) {
          hv = rope_f16x4_native(v, rope_entry(xs_lds + tbuf * XS * PLANE, lt, pidx));
        } else {
          hv = to_f16x4_native(v);
        }
        store_f16x4(p, orow, n, hv);
      } else if constexpr (EPI == Epi::F16) {
        store_f16x4(p, orow, n, to_f16x4_native(v));
      } else if constexpr (EPI == Epi::SWIGLU_F16) {
        *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(p.out) + orow * p.ldo + (n >> 1)) =
            swiglu_f16x2_native<true>(v);
      } else {
        store_out<EPI>(p, orow, n, v);
      }
    }
  }
}

template <int WF, int BT, int XS, Epi EPI, bool GROUPED, int NW = 4, int CT = 0, bool NORM = false, bool W16 = false>
void launch(pfhip_backend* b, const GemmArgs& a, const char* name) {
  constexpr int BN = NW * WF * 16;
  const int n_tiles = (a.N + BN - 1) / BN;
  const int t_tiles = GROUPED ? a.max_tiles : (a.M + BT - 1) / BT;
  const long grid = (long)n_tiles * t_tiles;
  if (grid == 0) return;
  PF_CHECK(grid < (1L << 31), "gemm_w4: grid too large");
  PF_CHECK(CT == 0 || a.K == CT * KC, "gemm_w4: K does not match the tile's compile-time chunk count");
  // activation buffers: two (double buffering) or all CT chunks, plus the
  // RoPE table's plane when every chunk buffer is taken
  constexpr int NBUF = CT > 0 ? (NORM ? 2 * CT : CT) + (EPI == Epi::ROPE_F16 ? 1 : 0) : 2;
  // (the top-k epilogue keeps 128 counters after the staged tile, and on the
  // 16-row tile the routing plan's 128 bitmaps, 256 offsets and 4 sums)
  const size_t lds = std::max((size_t)NBUF * XS * BT * KC * sizeof(uint16_t),
                              StagedOut<WF, BT, EPI, NW>::OK
                                  ? StagedOut<WF, BT, EPI, NW>::LDS + (EPI == Epi::F32_TOPK ? 516 * 4 : 0)
                                  : (size_t)0);
  auto go = [&](auto kern) {
    allow_lds(reinterpret_cast<const void*>(kern), lds);
    ProfScope ps(b, name);
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * NW), lds, b->stream, a);
    PF_HIP(hipGetLastError());
  };
  if (CT == 0 && (a.K / KC) % 2 == 0) go(&k_gemm_w4<WF, BT, XS, EPI, GROUPED, NW, CT, NORM, CT == 0, W16>);
  else go(&k_gemm_w4<WF, BT, XS, EPI, GROUPED, NW, CT, NORM, false, W16>);
}

template <int WF, int BT, int XS, bool GROUPED, int NW, int CT = 0>
void dispatch_epi(pfhip_backend* b, const GemmArgs& a, Epi epi, const char* name) {
  // the small tile (CT > 0) is built with one fragment per wave for every
  // epilogue and with two for the router's (N = 128 in one workgroup); the
  // all-K 64-row expert tile (grouped, five fragments) for the expert GEMMs
  constexpr bool ALL = CT == 0 || WF == 1 || (BT == 64 && WF == 5 && GROUPED);
  switch (epi) {
    case Epi::F16:
      if constexpr (ALL) return launch<WF, BT, XS, Epi::F16, GROUPED, NW, CT>(b, a, name);
      break;
    case Epi::F32: return launch<WF, BT, XS, Epi::F32, GROUPED, NW, CT>(b, a, name);
    case Epi::ROPE_F16:
      if constexpr (NW == 4 && ALL && !GROUPED) return launch<WF, BT, XS, Epi::ROPE_F16, GROUPED, NW, CT>(b, a, name);
      break;
    case Epi::SWIGLU_SPLIT: break;
    case Epi::SWIGLU_F16:
      if constexpr (ALL) return launch<WF, BT, XS, Epi::SWIGLU_F16, GROUPED, NW, CT>(b, a, name);
      break;
    case Epi::F32_TOPK:
      if constexpr (WF == 2 && (BT == 128 || BT == 64 || (BT == 16 && CT > 0)) && !GROUPED && NW == 4) {
        if constexpr ((CT == 0 && (BT == 64 || BT == 128)) || (CT == 5 && BT == 16))
          if (a.w16) return launch<WF, BT, XS, Epi::F32_TOPK, GROUPED, NW, CT, false, true>(b, a, name);
        return launch<WF, BT, XS, Epi::F32_TOPK, GROUPED, NW, CT>(b, a, name);
      }
      break;
  }
  throw Error("gemm_w4: unsupported epilogue for this tile");
}

template <int WF, int BT, int NW = 4, int CT = 0>
void dispatch_grouped(pfhip_backend* b, const GemmArgs& a, Epi epi, bool grouped, const char* name) {
  if (grouped) dispatch_epi<WF, BT, 1, true, NW, CT>(b, a, epi, name);
  else dispatch_epi<WF, BT, 1, false, NW, CT>(b, a, epi, name);
}

// 16-token tile with all of K loaded at once: K = 640 or 896 (5 or 7 chunks)
template <int WF>
void dispatch_small(pfhip_backend* b, const GemmArgs& a, Epi epi, bool grouped, const char* name) {
  if (a.nrm_res) {  // the router's residual add + norm on the way in
    if constexpr (WF == 2) {
      if (!grouped && a.K == 5 * KC && epi == Epi::F32_TOPK)
        return launch<2, 16, 1, Epi::F32_TOPK, false, 4, 5, true>(b, a, name);
      if (!grouped && a.K == 5 * KC && epi == Epi::F32) return launch<2, 16, 1, Epi::F32, false, 4, 5, true>(b, a, name);
    }
    throw Error("gemm_w4: the input norm is built for the 16-token router tile, K = 640");
  }
  switch (a.K / KC) {
    case 5: return dispatch_grouped<WF, 16, 4, 5>(b, a, epi, grouped, name);
    case 7: return dispatch_grouped<WF, 16, 4, 7>(b, a, epi, grouped, name);
    default: throw Error("gemm_w4: the 16-token tile is built for K = 640 and 896");
  }
}

// ---------------------------------------------------------------- weight prep

// MatMulNBits bytes [G][N][K/2] (nibble k at bits 4k of the dword of 8
// values) -> repacked dwords: value k at bits 8k (k < 4) or 8(k-4)+4.
__global__ void k_w4_repack(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint32_t w = src[i];
  uint32_t r = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t q = (w >> (4 * k)) & 0xFu;
    r |= q << (k < 4 ? 8 * k : 8 * (k - 4) + 4);
  }
  dst[i] = r;
}

// fp16 scales [G][N][nb] + packed zero-points [G][N][ceil(nb/2)] (NULL = 0)
// -> per block: low half fp16 -(1024 + zp), high half the fp16 scale.
__global__ void k_w4_scale_pairs(const uint16_t* __restrict__ ws, const uint8_t* __restrict__ wz,
                                 uint32_t* __restrict__ out, int rows, int nb) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)rows * nb) return;
  const size_t row = i / nb;
  const int blk = (int)(i % nb);
  uint32_t zp = 0;
  if (wz) {
    const uint8_t zb = wz[row * ((nb + 1) >> 1) + (blk >> 1)];
    zp = (blk & 1) ? (zb >> 4) : (zb & 0xFu);
  }
  const _Float16 off = (_Float16)(-(1024.0f + (float)zp));
  out[i] = (uint32_t)__builtin_bit_cast(uint16_t, off) | ((uint32_t)ws[i] << 16);
}

}  // namespace

void gemm_w4(pfhip_backend* b, const GemmArgs& a, XKind xk, Epi epi, bool grouped, int tile_t, int wf,
             const char* prof_name) {
  PF_CHECK(a.K > 0 && a.K % KC == 0, "gemm_w4: K must be a positive multiple of 128");
  PF_CHECK(a.N > 0, "gemm_w4: N must be positive");
  PF_CHECK(a.x && ((a.w && a.wsz) || a.w16) && (a.out || epi == Epi::F32_TOPK || a.out_f32w), "gemm_w4: null operand");
  if (a.out_f32w) PF_CHECK(epi == Epi::F16 && !grouped, "gemm_w4: the widened f32 output is for the dense F16 epilogue");
  if (a.w16)
    PF_CHECK(epi == Epi::F32_TOPK && !grouped && (tile_t == 64 || tile_t == 128 || (tile_t == 16 && a.K == 5 * KC)) &&
                 wf == 2 && !a.nrm_res && (reinterpret_cast<uintptr_t>(a.w16) & 15) == 0 &&
                 (long)a.N * a.K * 2 < (1L << 31),
             "gemm_w4: fp16 weights are built for the router top-k tile (16 rows with K = 640, 64 or 128 rows), "
             "16-byte aligned");
  PF_CHECK(a.ldx % 8 == 0, "gemm_w4: activation row stride must allow 16-byte loads");
  PF_CHECK((reinterpret_cast<uintptr_t>(a.x) & 15) == 0 && (reinterpret_cast<uintptr_t>(a.w) & 15) == 0,
           "gemm_w4: activations and weights must be 16-byte aligned");  // (w is null with fp16 weights)
  // activation rows are addressed with 32-bit element offsets (grouped: a.M
  // slots bound every row the tile list or the row map can name)
  PF_CHECK((long)a.M * a.ldx < (1L << 31), "gemm_w4: activation offsets exceed 32 bits");
  // the weight and scale-pair buffer descriptors hold one matrix (expert) of N x K values
  PF_CHECK((long)a.N * a.K / 2 < (1L << 31), "gemm_w4: one weight matrix must stay below 2^31 bytes");
  if (xk == XKind::SPLIT)
    PF_CHECK(a.x_lo && (reinterpret_cast<uintptr_t>(a.x_lo) & 15) == 0, "gemm_w4: SPLIT needs an aligned lo plane");
  if (epi == Epi::SWIGLU_SPLIT || epi == Epi::SWIGLU_F16) PF_CHECK(a.N % 4 == 0, "gemm_w4: SwiGLU needs N % 4 == 0");
  if (epi == Epi::SWIGLU_SPLIT) PF_CHECK(a.out_lo, "gemm_w4: SWIGLU_SPLIT needs an output lo plane");
  if (epi == Epi::ROPE_F16)
    PF_CHECK(a.rope_pairs && (reinterpret_cast<uintptr_t>(a.rope_pairs) & 15) == 0 && a.seq_len > 0 &&
                 a.rope_cols % 64 == 0,
             "gemm_w4: RoPE epilogue needs an aligned fp16 pair table, seq_len and head-aligned rope_cols");
  if (epi == Epi::ROPE_F16) PF_CHECK(!grouped && (long)a.M < (1L << 31), "RoPE epilogue: dense rows below 2^31");
  if (grouped) PF_CHECK(a.tiles && a.num_tiles && a.max_tiles > 0, "gemm_w4: grouped mode needs a tile list");
  else PF_CHECK(a.M >= 0, "gemm_w4: M must be non-negative");
  PF_CHECK(xk == XKind::F16, "gemm_w4: activations must be one fp16 plane");
  // staged (whole-line) output stores need 16-byte aligned rows and no
  // partial 16-byte unit at column N
  GemmArgs g = a;
  {
    const int esz = epi == Epi::F32 || epi == Epi::F32_TOPK ? 4 : 2;
    const int ocols = epi == Epi::SWIGLU_F16 ? a.N / 2 : a.N;
    g.out_staged = (epi == Epi::F32 || epi == Epi::F32_TOPK || epi == Epi::F16 || epi == Epi::ROPE_F16 ||
                    epi == Epi::SWIGLU_F16) &&
                   ocols % (16 / esz) == 0 && (a.ldo * esz) % 16 == 0 &&
                   (reinterpret_cast<uintptr_t>(a.out) & 15) == 0 && (epi != Epi::SWIGLU_F16 || a.N % 16 == 0) &&
                   !a.out_f32w;
  }
  PF_CHECK(epi != Epi::SWIGLU_SPLIT, "gemm_w4: SwiGLU output is fp16");
  if (epi == Epi::F32_TOPK)
    PF_CHECK(!grouped && (tile_t == 128 || tile_t == 64 || tile_t == 16) && wf == 2 && a.N == 128 && a.topk_k == 4 &&
                 a.topk_idx &&
                 a.topk_w && g.out_staged,
             "gemm_w4: the top-k epilogue needs N == 128, K == 4, a 128- or 16-token tile of 128 columns and "
             "16-byte aligned f32 rows");
  if (a.plan_slot_of)
    PF_CHECK(epi == Epi::F32_TOPK && tile_t == 16 && a.M >= 1 && a.M <= 16 && a.plan_expert_off && a.plan_slot_token &&
                 a.plan_tiles && a.plan_num_tiles && a.plan_tile_t >= 1,
             "gemm_w4: the routing plan is built by the single 16-row router tile (M <= 16), with every plan output");
  if (tile_t == 128 && wf == 4) return dispatch_grouped<4, 128>(b, g, epi, grouped, prof_name);
  // 64-row expert tiles with K = 640 load all five chunks at once (80 KB of
  // LDS, two workgroups per CU): a tile waits for memory once instead of
  // once per chunk, which is what bounds these GEMMs at a few hundred tiles
  if (tile_t == 64 && wf == 5 && grouped && a.K == 5 * KC)
    return dispatch_epi<5, 64, 1, true, 4, 5>(b, g, epi, prof_name);
  if (tile_t == 64 && wf == 5) return dispatch_grouped<5, 64>(b, g, epi, grouped, prof_name);
  if (tile_t == 128 && wf == 2) return dispatch_grouped<2, 128>(b, g, epi, grouped, prof_name);
  if (tile_t == 64 && wf == 2) return dispatch_grouped<2, 64>(b, g, epi, grouped, prof_name);
  if (tile_t == 64 && wf == 1) return dispatch_grouped<1, 64>(b, g, epi, grouped, prof_name);
  if (a.nrm_res)
    PF_CHECK(a.nrm_gamma && a.nrm_h && a.nrm_xn && a.ldx == a.K && tile_t == 16 &&
                 ((reinterpret_cast<uintptr_t>(a.nrm_res) | reinterpret_cast<uintptr_t>(a.nrm_gamma) |
                   reinterpret_cast<uintptr_t>(a.nrm_h) | reinterpret_cast<uintptr_t>(a.nrm_xn)) & 15) == 0,
             "gemm_w4: input norm needs residual, gamma and outputs (16-byte aligned, rows of K) on the 16-token tile");
  if (tile_t == 16 && wf == 1) return dispatch_small<1>(b, g, epi, grouped, prof_name);
  if (tile_t == 16 && wf == 2) return dispatch_small<2>(b, g, epi, grouped, prof_name);
  throw Error("gemm_w4: unsupported (tile_t, wf) = (" + std::to_string(tile_t) + ", " + std::to_string(wf) + ")");
}

// ---------------------------------------------------------------- O GEMM + residual + RMSNorm
//
// The attention output projection with the block's post-attention residual
// add and RMSNorm fused into the epilogue (the O MatMulNBits, add_fp16 and
// add_rmsnorm_fp16_to_f32 of zig/wasm_exports.zig:560-707, 969-990,
// 288-350, in the GPU shaders' fp16 numerics):
//   o   = fp16(x . w16^T + bias)                      (the GEMM output)
//   h2  = fp16(o + h)                                 (the new residual)
//   xn  = fp16(h2 / sqrt(mean((o + h)^2) + eps) * g)  (sum of squares of the
//         unrounded f32 sum, normalising the rounded one)
// A workgroup of 8 waves owns 64 whole rows (all N = 8 x 5 x 16 = 640
// columns), so the row's sum of squares is reduced in the workgroup (lanes,
// then waves through LDS) and o never goes to memory.
namespace {

constexpr int RN_NW = 8, RN_WF = 5, RN_BT = 64;
constexpr int RN_BN = RN_NW * RN_WF * 16;  // 640
// chunks loaded ahead of the one computed, and activation buffers: two
// ahead for 64-row tiles; one for 128-row tiles, whose chunks carry twice
// the MFMAs. (128-row tiles do not fit: 160 accumulator registers plus the
// weight sets and addresses exceed 256 and spill.)
constexpr int RN_PD = RN_BT <= 64 ? 2 : 1;
constexpr int RN_NB = RN_PD + 1;
// The residual tile (BT rows x 640 fp16) is copied into LDS behind the
// activation buffers while the last chunks are computed: RN_RESC 16-byte
// copies per lane, rows of 80 units whose unit u sits at slot u ^ (row & 15)
// (XOR within aligned 16-unit blocks, so the 16 rows a wave reads at once
// fall in distinct banks).
constexpr int RN_RESC = RN_BT * RN_BN * 2 / 16 / (64 * RN_NW);
static_assert(RN_BT * RN_BN * 2 % (16 * 64 * RN_NW) == 0 && RN_BN % 128 == 0, "whole residual copies");
constexpr size_t RN_LDS = (size_t)RN_NB * RN_BT * KC * 2 + (size_t)RN_BT * RN_BN * 2;

// copy16_to_lds issued as inline assembly: the compiler then does not know
// that it writes LDS and does not make every workgroup barrier wait for all
// such copies in flight (vmcnt(0)); the kernel waits for the ones it needs
// itself. Clobbers M0, which nothing else in the kernel uses. An LDS DMA
// reads M0 one wait state after the write at the earliest (the s_nop).
__device__ __forceinline__ void copy16_to_lds_async(const void* src, uint32_t lds_byte) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(src), "s"(lds_byte)
               : "memory", "m0");
}

// C = K / 128 chunks, fully unrolled: chunk c + 2 is loaded while chunk c
// is computed (three activation buffers, three weight register sets), so a
// load has two chunks of MFMAs to land; with one 8-wave workgroup per CU
// nothing else hides it.
template <int C>
__global__ __launch_bounds__(64 * RN_NW, 1) void k_gemm_w4_rownorm(GemmArgs p, const uint16_t* __restrict__ resid,
                                                                   const uint16_t* __restrict__ gamma,
                                                                   uint16_t* __restrict__ h_out,
                                                                   uint16_t* __restrict__ xn_out, float eps) {
  constexpr int NW8 = RN_NW, WF = RN_WF, BT = RN_BT, TJ = BT / 16;
  constexpr int XI = BT * KC * 2 / 1024 / NW8;  // 1 KB direct loads per wave per chunk
  constexpr int PLANE = BT * KC;                // halves per buffer
  static_assert(XI >= 1 && BT * KC * 2 % (1024 * NW8) == 0, "whole 1 KB copies per wave");
  // vector memory instructions per lane and chunk, issued in this order:
  // WF weight and WF scale loads, then XI activation copies
  constexpr int VM_PER_CHUNK = 2 * WF + XI;
  constexpr int PD = RN_PD, NB = RN_NB;
  // the residual copies are issued in chunk C0's iteration, after the last chunk's loads
  constexpr int C0 = C - 1 - PD;
  static_assert(C0 >= 0, "residual copies after the last chunk's loads");
  // [NB][BT][KC] swizzled activations (then the row sums), then [BT][640] residual
  extern __shared__ __attribute__((aligned(16))) _Float16 xs_lds[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const int tt = xcd_remap(blockIdx.x, gridDim.x);
  const int row0 = tt * BT;
  const int rows = min(BT, p.M - row0);
  if (rows <= 0) return;
  const int kd = p.K >> 3, nb = p.K >> 5;

  const uint32_t* __restrict__ W = reinterpret_cast<const uint32_t*>(p.w);
  const uint32_t* wptr[WF];
  const uint32_t* sptr[WF];
#pragma unroll
  for (int f = 0; f < WF; ++f) {
    const int n = (wave * WF + f) * 16 + l16;
    wptr[f] = W + (size_t)n * kd + lg * 4;
    sptr[f] = p.wsz + (size_t)n * nb + lg;
  }
  const uint16_t* __restrict__ xsrc = static_cast<const uint16_t*>(p.x);
  int xoff[XI];
#pragma unroll
  for (int m = 0; m < XI; ++m) {
    const int r = (m * NW8 + wave) * 4 + lg;
    xoff[m] = (row0 + min(r, rows - 1)) * p.ldx + ((l16 ^ (r & 15)) << 3);
  }
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_ptr_t)xs_lds;
  auto load_x = [&](int c, int buf) {
#pragma unroll
    for (int m = 0; m < XI; ++m)
      copy16_to_lds_async(xsrc + xoff[m] + c * KC,
                          __builtin_amdgcn_readfirstlane(lds0 + (uint32_t)(buf * PLANE + (m * NW8 + wave) * 512) * 2));
  };
  const uint32_t res_lds = lds0 + (uint32_t)(NB * PLANE) * 2;
  auto load_res_lds = [&]() {
#pragma unroll
    for (int i = 0; i < RN_RESC; ++i) {
      const int u = (i * NW8 + wave) * 64 + lane;  // LDS unit of this lane's copy
      const int t = u / (RN_BN / 8), slot = u % (RN_BN / 8);
      const int g = slot ^ (t & 15);               // the row's unit held there
      copy16_to_lds_async(resid + (size_t)(row0 + min(t, rows - 1)) * RN_BN + g * 8,
                          __builtin_amdgcn_readfirstlane(res_lds + (uint32_t)((i * NW8 + wave) * 64) * 16));
    }
  };
  u4_t wraw[C][WF];  // only PD + 1 chunks' sets are live at a time
  uint32_t sz[C][WF];
  auto load_w = [&](int c) {
#pragma unroll
    for (int f = 0; f < WF; ++f) {
      wraw[c][f] = *reinterpret_cast<const u4_t*>(wptr[f] + c * 16);
      sz[c][f] = sptr[f][c * 4];
    }
  };

  int ncol[WF];
#pragma unroll
  for (int f = 0; f < WF; ++f) ncol[f] = (wave * WF + f) * 16 + 4 * lg;
  // the bias is loaded before the first chunks and widened after they are
  // issued, so that its latency overlaps theirs
  u2_t braw[WF];
#pragma unroll
  for (int f = 0; f < WF; ++f) braw[f] = p.bias ? *reinterpret_cast<const u2_t*>(p.bias + ncol[f]) : u2_t{0u, 0u};
  f4_t acc[WF][TJ];

  auto compute = [&](int c) {
    h2_t off[WF], offh[WF], sc[WF];
#pragma unroll
    for (int f = 0; f < WF; ++f) {
      const h2_t pr = __builtin_bit_cast(h2_t, sz[c][f]);
      off[f] = h2_t{pr.x, pr.x};
      offh[f] = off_high(off[f]);
      sc[f] = h2_t{pr.y, pr.y};
    }
    const _Float16* xb = xs_lds + (c % NB) * PLANE;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      h8_t wd[WF];
#pragma unroll
      for (int f = 0; f < WF; ++f) wd[f] = dequant_fold(wraw[c][f][j], off[f], offh[f], sc[f]);
      const int unit = ((4 * lg + j) ^ l16) << 3;
#pragma unroll
      for (int tj = 0; tj < TJ; ++tj) {
        const h8_t xh = *reinterpret_cast<const h8_t*>(xb + (16 * tj + l16) * KC + unit);
#pragma unroll
        for (int f = 0; f < WF; ++f) acc[f][tj] = mfma16x16x32(wd[f], xh, acc[f][tj]);
      }
    }
  };

#pragma unroll
  for (int i = 0; i < PD && i < C; ++i) {
    load_w(i);
    load_x(i, i);
  }
#pragma unroll
  for (int f = 0; f < WF; ++f) {
    // the bias widens as k_gemm_w4 widens it (the two O forms agree bit for bit)
    const uint32_t bwv[2] = {braw[f].x, braw[f].y};
    float bv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) bv[r] = (float)__builtin_bit_cast(_Float16, (uint16_t)(bwv[r >> 1] >> (16 * (r & 1))));
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[f][j] = f4_t{bv[0], bv[1], bv[2], bv[3]};
  }
#pragma unroll
  for (int c = 0; c < C; ++c) {
    // nothing moves between chunks (the compiler's own waits for the weight
    // registers do not count the copies, so hoisting chunk c + 1's dequant
    // into chunk c would make it wait for copies just issued)
    __builtin_amdgcn_sched_barrier(0);
    // This wave's copies of chunk c have landed once no more vector memory
    // instructions are outstanding than were issued after them: those of
    // chunks c + 1 .. c + PD - 1 (s_waitcnt: vmcnt in bits 3:0 and 15:14;
    // expcnt and lgkmcnt at their maxima, i.e. not waited on).
    // The residual copies, issued after chunk C - 1's loads, may stay in
    // flight until the epilogue.
    static_assert(VM_PER_CHUNK + RN_RESC < 64 && PD <= 2, "vmcnt is 6 bits");
    constexpr int VR = VM_PER_CHUNK + RN_RESC;
    if (PD == 2 && c + 1 < C && c <= C0) {
      __builtin_amdgcn_s_waitcnt((VM_PER_CHUNK & 15) | (7 << 4) | (15 << 8) | ((VM_PER_CHUNK >> 4) << 14));
    } else if (PD == 2 && c + 1 < C) {
      __builtin_amdgcn_s_waitcnt((VR & 15) | (7 << 4) | (15 << 8) | ((VR >> 4) << 14));
    } else if (c > C0) {
      __builtin_amdgcn_s_waitcnt((RN_RESC & 15) | (7 << 4) | (15 << 8) | ((RN_RESC >> 4) << 14));
    } else {
      __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
    }
    // every wave's copies too; and buffer (c + PD) % NB was last read by
    // compute(c - 1). The fences are LDS-only: __syncthreads' full fence
    // would also wait for the weight loads of the chunks in flight.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    if (c + PD < C) {
      load_w(c + PD);
      load_x(c + PD, (c + PD) % NB);
    }
    if (c == C0) load_res_lds();
    compute(c);
  }
  __builtin_amdgcn_sched_barrier(0);
  // every wave's residual copies have landed
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");

  // ---- epilogue: lane holds o[token 16 tj + l16][ncol[f] .. + 3]
  u2_t gw[WF];
#pragma unroll
  for (int f = 0; f < WF; ++f) gw[f] = *reinterpret_cast<const u2_t*>(gamma + ncol[f]);
  u2_t hs[WF][TJ];   // h2 (fp16)
  float ss[TJ];
  // residual rows from LDS, one token fragment ahead
  // (h2, then xn, are written over the residual in the same layout and
  // leave as whole rows)
  char* res_tile = reinterpret_cast<char*>(xs_lds) + NB * PLANE * 2;
  auto res_at = [&](int tj, int f) -> u2_t* {
    const int t = 16 * tj + l16;  // rows past the tile hold copies of the last (never stored)
    const int u = ncol[f] >> 3;   // 16-byte unit; the lane's 8 bytes are its half 4 lg & 4
    return reinterpret_cast<u2_t*>(res_tile + t * (RN_BN * 2) + ((u ^ (t & 15)) << 4) + (ncol[f] & 4) * 2);
  };
  u2_t rres[2][WF];
  auto load_res = [&](int tj, u2_t (&dst)[WF]) {
#pragma unroll
    for (int f = 0; f < WF; ++f) dst[f] = *res_at(tj, f);
  };
  // the tile's rows from LDS to dst: unit slot U of the tile is unit
  // (U % 80) ^ (row & 15) of row U / 80
  auto store_rows = [&](uint16_t* __restrict__ dst) {
#pragma unroll
    for (int i = 0; i < RN_RESC; ++i) {
      const int U = i * 64 * NW8 + tid;
      const int t = U / (RN_BN / 8), slot = U % (RN_BN / 8);
      if (t < rows)
        *reinterpret_cast<u4_t*>(dst + (size_t)(row0 + t) * RN_BN + (slot ^ (t & 15)) * 8) =
            *reinterpret_cast<const u4_t*>(res_tile + U * 16);
    }
  };
  load_res(0, rres[0]);
#pragma unroll
  for (int tj = 0; tj < TJ; ++tj) {
    if (tj + 1 < TJ) load_res(tj + 1, rres[(tj + 1) & 1]);
    ss[tj] = 0.0f;
#pragma unroll
    for (int f = 0; f < WF; ++f) {
      const float ov[4] = {acc[f][tj][0], acc[f][tj][1], acc[f][tj][2], acc[f][tj][3]};
      const h4_t o16 = __builtin_bit_cast(h4_t, to_f16x4_native(ov));
      const h4_t r16 = __builtin_bit_cast(h4_t, rres[tj & 1][f]);
      float sv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sv[r] = (float)o16[r] + (float)r16[r];
        ss[tj] = fmaf(sv[r], sv[r], ss[tj]);
      }
      hs[f][tj] = to_f16x4_native(sv);
      *res_at(tj, f) = hs[f][tj];  // over the residual this lane read
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  // row sums of squares: the 4 lane groups, then the 8 waves (fixed order)
  float* red = reinterpret_cast<float*>(xs_lds);  // [NW8][BT]
  __syncthreads();  // every wave is done with the activation buffers, and h2 is in LDS
#pragma unroll
  for (int tj = 0; tj < TJ; ++tj) {
    float v = ss[tj];
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    if (lg == 0) red[wave * BT + 16 * tj + l16] = v;
  }
  store_rows(h_out);
  __syncthreads();  // the row sums are written and every h2 unit is read
#pragma unroll
  for (int tj = 0; tj < TJ; ++tj) {
    const int t = 16 * tj + l16;
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < NW8; ++w) tot += red[w * BT + t];
    const float inv_rms = 1.0f / sqrtf(tot * (1.0f / (float)RN_BN) + eps);
#pragma unroll
    for (int f = 0; f < WF; ++f) {
      const h4_t hv = __builtin_bit_cast(h4_t, hs[f][tj]);
      const h4_t gm = __builtin_bit_cast(h4_t, gw[f]);
      float y[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) y[r] = (float)hv[r] * inv_rms * (float)gm[r];
      *res_at(tj, f) = to_f16x4_native(y);
    }
  }
  __syncthreads();
  store_rows(xn_out);
}

}  // namespace

void gemm_w4_add_rmsnorm(pfhip_backend* b, const GemmArgs& a, const uint16_t* resid, const uint16_t* gamma,
                         uint16_t* h_out, uint16_t* xn_out, float eps) {
  PF_CHECK(a.N == RN_BN, "gemm_w4_add_rmsnorm: N must be 640 (one workgroup per whole row)");
  PF_CHECK(a.K > 0 && a.K % KC == 0, "gemm_w4_add_rmsnorm: K must be a positive multiple of 128");
  PF_CHECK(a.x && a.w && a.wsz && resid && gamma && h_out && xn_out, "gemm_w4_add_rmsnorm: null operand");
  PF_CHECK(a.ldx % 8 == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 &&
               (reinterpret_cast<uintptr_t>(a.w) & 15) == 0,
           "gemm_w4_add_rmsnorm: activations and weights must be 16-byte aligned");
  PF_CHECK((reinterpret_cast<uintptr_t>(resid) & 15) == 0, "gemm_w4_add_rmsnorm: residual must be 16-byte aligned");
  PF_CHECK(((reinterpret_cast<uintptr_t>(resid) | reinterpret_cast<uintptr_t>(gamma) |
             reinterpret_cast<uintptr_t>(h_out) | reinterpret_cast<uintptr_t>(xn_out) |
             reinterpret_cast<uintptr_t>(a.bias)) & 7) == 0,
           "gemm_w4_add_rmsnorm: residual, gamma, bias and outputs must be 8-byte aligned");
  PF_CHECK(a.M >= 0 && (long)a.M * a.ldx < (1L << 31), "gemm_w4_add_rmsnorm: activation offsets exceed 32 bits");
  if (a.M == 0) return;
  const int grid = (a.M + RN_BT - 1) / RN_BT;
  static_assert((size_t)RN_NW * RN_BT * sizeof(float) <= (size_t)RN_NB * RN_BT * KC * 2, "row sums fit the buffers");
  const size_t lds = RN_LDS;
  auto go = [&](auto kern) {
    allow_lds(reinterpret_cast<const void*>(kern), lds);
    ProfScope ps(b, "gemm_o_add_rmsnorm");
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * RN_NW), lds, b->stream, a, resid, gamma, h_out,
                       xn_out, eps);
    PF_HIP(hipGetLastError());
  };
  switch (a.K / KC) {
    case 5: return go(&k_gemm_w4_rownorm<5>);
    case 7: return go(&k_gemm_w4_rownorm<7>);
    default: throw Error("gemm_w4_add_rmsnorm: K must be 640 or 896");
  }
}

void w4_prepare(pfhip_backend* b, const uint8_t* w, const uint16_t* ws, const uint8_t* wz, uint32_t* w_out,
                uint32_t* sz_out, int rows, int K) {
  PF_CHECK(rows > 0 && K > 0 && K % 32 == 0, "w4_prepare: bad shape");
  PF_CHECK((reinterpret_cast<uintptr_t>(w) & 3) == 0, "w4_prepare: weights must be 4-byte aligned");
  const size_t nd = (size_t)rows * (K / 8);
  const int nb = K / 32;
  ProfScope ps(b, "w4_prepare");
  hipLaunchKernelGGL(k_w4_repack, dim3((unsigned)((nd + 255) / 256)), dim3(256), 0, b->stream,
                     reinterpret_cast<const uint32_t*>(w), w_out, nd);
  PF_HIP(hipGetLastError());
  const size_t ns = (size_t)rows * nb;
  hipLaunchKernelGGL(k_w4_scale_pairs, dim3((unsigned)((ns + 255) / 256)), dim3(256), 0, b->stream, ws, wz, sz_out,
                     rows, nb);
  PF_HIP(hipGetLastError());
}

}  // namespace pf
