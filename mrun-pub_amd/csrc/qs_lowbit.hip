// Packed int3 / int2 QStore GEMV and dequant on gfx950.
//
// Layout (reference qstore_int3.py:30-56, qstore_int2.py:24-63): every weight row is an
// LSB-first bitstream, code k at bits [b*k, b*k + b) of the row, row_bytes =
// ceil(K*b/8); one scale per (row, group of G codes).  Weight value
//   w[n,k] = (float(code) - zero[n, k/G]) * scale[n, k/G]
// with zero the reference's fixed offset (4 for int3, 1 for int2; scales fp32, G = 128) or
// a per-group zero point (fp16 scale + fp16 zero, G = 64: the asymmetric variant).
//
// All GEMV kernels compute y[m,n] = sum_k x[m,k] w[n,k] in fp32 the same way: codes are
// widened to the exact bf16 values OFF + code (OFF = 8 for 3-bit, 4 for 2-bit: bf16 bit
// pattern 0x4100 | code << 4, resp. 0x4080 | code << 5 -- one bfe, one 24-bit multiply and
// one v_bitop3 per PAIR of codes) and multiplied with bf16 activations (products exact
// in fp32); per group (or any piece of a group)
//   sum_k x (code - z) = R - (OFF + z) * S0,     S0 = sum_{k in group} x[m,k],
// and y += scale * (R - (OFF + z) * S0).  fp32 activations are split exactly into three
// bf16 terms (x = h + m + l) that run as three activation rows and are summed at the end.
//   k_lowbit_valu  decode (M <= 2 bf16 rows): one wave per weight row, v_dot2_f32_bf16
//   k_lowbit_gk    3..16 bf16 rows, one launch: v_mfma_f32_16x16x32_bf16 per group, a
//                  quarter group per lane, K split over the waves of a workgroup
//   k_lowbit_slot  M <= 16 fp32 rows (split into bf16 terms): one whole group per lane
//   k_lowbit_mfma  any aligned-to-4 layout (fallback), four lanes per group
//   k_lowbit_any   every other layout (any group size, a short last group, unaligned
//                  rows): one wave per weight row, scalar decode
#include "qs_common.h"

#include <limits.h>

namespace qs {

struct LowbitParams {
  const uint16_t* x;   // bf16 [M, K] (M <= 16)
  int64_t ldx;
  const float* s0;     // [M, ng] group sums of x
  const uint8_t* packed;
  int64_t row_bytes;
  const void* scales;  // [N, ng] f32 or f16
  const void* zeros;   // [N, ng] f16/f32, nullable
  int scale_f16, zero_f16;
  float offset;        // used when zeros == nullptr
  float* y;            // [M, N]
  int64_t ldy;
  int M, N, K, ng;
  uint32_t pair_mask, pair_base;  // code-pair -> bf16x2 (OFF + c) masks, set by pair_consts()
};

// (t * spread) & mask | base turns the 2*BITS-bit code pair t into two bf16 (OFF + c).
// mask/base travel as kernel arguments (scalar registers) so that the and/or is a single
// v_bitop3_b32 (table 0xEA = (a & b) | c).
template <int BITS>
__device__ __forceinline__ uint32_t pair_bf16(uint32_t t, uint32_t mask, uint32_t base) {
  constexpr uint32_t spread = BITS == 3 ? 0x20010u : 0x80020u;
  return __builtin_amdgcn_bitop3_b32(t * spread, mask, base, 0xEA);
}

inline void pair_consts(LowbitParams& p, int bits) {
  p.pair_mask = bits == 3 ? 0x00700070u : 0x00600060u;
  p.pair_base = bits == 3 ? 0x41004100u : 0x40804080u;
}

// Lane code extraction: the lane's G/4 codes (BITS*G/4 bits, at a 2- or 4-byte aligned
// offset) are returned as a 64/96-bit little-endian field.
// Weight-stream load: nontemporal (the M <= 2 decode kernels, measured faster so) or plain
// (the multi-row kernels, measured faster so).
template <bool NT, typename T>
__device__ __forceinline__ T ldw(const T* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}

template <int BITS, int G, bool NT = true>
__device__ __forceinline__ void load_codes(const uint8_t* p, uint32_t (&f)[3]) {
  constexpr int NB = BITS * G / 4;  // bits per lane: 48, 96, 32, 64
  if constexpr (NB == 96) {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
    f[0] = ldw<NT>(q);
    f[1] = ldw<NT>(q + 1);
    f[2] = ldw<NT>(q + 2);
  } else if constexpr (NB == 64) {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
    f[0] = ldw<NT>(q);
    f[1] = ldw<NT>(q + 1);
    f[2] = 0;
  } else if constexpr (NB == 32) {
    f[0] = ldw<NT>(reinterpret_cast<const uint32_t*>(p));
    f[1] = f[2] = 0;
  } else {  // 48 bits at a 2-byte aligned offset; never reads outside [p, p + 6)
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    if (a & 2) {
      const uint16_t h0 = ldw<NT>(reinterpret_cast<const uint16_t*>(p));
      const uint32_t d1 = ldw<NT>(reinterpret_cast<const uint32_t*>(p + 2));
      f[0] = (uint32_t)h0 | (d1 << 16);
      f[1] = d1 >> 16;
    } else {
      f[0] = ldw<NT>(reinterpret_cast<const uint32_t*>(p));
      f[1] = ldw<NT>(reinterpret_cast<const uint16_t*>(p + 4));
    }
    f[2] = 0;
  }
}

// 2 codes starting at bit position bp of the field -> packed bf16 pair (OFF + c).
template <int BITS>
__device__ __forceinline__ uint32_t code_pair(const uint32_t (&f)[3], int bp, uint32_t mask, uint32_t base) {
  const int w = bp >> 5, o = bp & 31;
  uint32_t t;
  if (o + 2 * BITS <= 32)
    t = __builtin_amdgcn_ubfe(f[w], o, 2 * BITS);
  else
    t = __builtin_amdgcn_ubfe(__builtin_amdgcn_alignbit(f[w + 1], f[w], o), 0, 2 * BITS);
  return pair_bf16<BITS>(t, mask, base);  // int3: 8 + c at bits 4-6 / 20-22; int2: 4 + c at 5-6 / 21-22
}

template <int BITS, int G, int KW>
__global__ __launch_bounds__(KW * 64) void k_lowbit_mfma(LowbitParams p) {
  constexpr int CODES = G / 4;               // codes per lane per group
  constexpr int CB = BITS * G / 8;           // bytes per row per group
  constexpr int LB = BITS * CODES / 8;       // bytes per lane per group (may be 6)
  constexpr int NMMA = G / 32;               // MFMAs per group
  constexpr float OFF = BITS == 3 ? 8.f : 4.f;
  const int lane = threadIdx.x & 63;
  const int ks = threadIdx.x >> 6;
  const int col = lane & 15, g4 = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int n = min(n0 + col, p.N - 1);
  const uint8_t* row = p.packed + (int64_t)n * p.row_bytes + g4 * LB;
  const bool mval = col < p.M;
  const uint16_t* xr = p.x + (int64_t)(mval ? col : 0) * p.ldx + g4 * CODES;
  f32x4 y = {0.f, 0.f, 0.f, 0.f};

  // UG groups per round: their codes, activations and scales are all requested before
  // the first one is consumed.
  constexpr int UG = 4;
  for (int g0 = ks; g0 < p.ng; g0 += UG * KW) {
    uint32_t f[UG][3];
    bf16x8 xa[UG][NMMA];
    float sc[UG], z[UG];
#pragma unroll
    for (int u = 0; u < UG; ++u) {
      const int g = g0 + u * KW;
      if (g < p.ng) {
        load_codes<BITS, G>(row + (int64_t)g * CB, f[u]);
#pragma unroll
        for (int j = 0; j < NMMA; ++j)
          xa[u][j] = mval ? *reinterpret_cast<const bf16x8*>(xr + (int64_t)g * G + 8 * j) : bf16x8{};
        const int64_t si = (int64_t)n * p.ng + g;
        sc[u] = p.scale_f16 ? f16_bits_to_f32(static_cast<const uint16_t*>(p.scales)[si])
                            : static_cast<const float*>(p.scales)[si];
        if (p.zeros)
          z[u] = p.zero_f16 ? f16_bits_to_f32(static_cast<const uint16_t*>(p.zeros)[si])
                            : static_cast<const float*>(p.zeros)[si];
        else
          z[u] = p.offset;
      }
    }
#pragma unroll
    for (int u = 0; u < UG; ++u) {
      const int g = g0 + u * KW;
      if (g >= p.ng) break;
      f32x4 r = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NMMA; ++j) {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        u32x4 b;
#pragma unroll
        for (int d = 0; d < 4; ++d) b[d] = code_pair<BITS>(f[u], BITS * (8 * j + 2 * d), p.pair_mask, p.pair_base);
        r = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[u][j], __builtin_bit_cast(bf16x8, b), r, 0, 0, 0);
      }
      const float c = OFF + z[u];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = 4 * g4 + q;
        const float s0 = m < p.M ? p.s0[(int64_t)m * p.ng + g] : 0.f;
        y[q] = fmaf(sc[u], fmaf(-c, s0, r[q]), y[q]);
      }
    }
  }
  __shared__ f32x4 red[KW][64];
  red[ks][lane] = y;
  __syncthreads();
  if (ks != 0) return;
  f32x4 t = red[0][lane];
#pragma unroll
  for (int w = 1; w < KW; ++w) t += red[w][lane];
  const int no = n0 + col;
  if (no >= p.N) return;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int m = 4 * g4 + q;
    if (m < p.M) p.y[(int64_t)m * p.ldy + no] = t[q];
  }
}

// ----------------------------------------------------------------------------------
// Slotted GEMV (k_lowbit_slot): the per-group MFMA formulation with one WHOLE group per
// lane, so that a lane reads its codes as contiguous 8-byte words and many groups are in
// flight per wave.  Wave = 16 weight rows (lane l: row l & 15, slot l >> 4).  Step t covers
// the groups gb = 4t .. 4t+3 of the workgroup's range; slot s holds the CB code bytes of
// group gb + s of its row (B operand: 8 codes per MFMA, G/8 MFMAs per group).  The A
// operand keeps the four groups apart: A row i = 4*mi + slot carries activation row mi
// only in the k-block of that slot (zeros elsewhere), so D[4*mi + q][n] is the sum over
// group gb + q alone and
//   y[m, n] += scale[n, gb+q] * (D - (OFF + zero[n, gb+q]) * S0[m, gb+q]).
// Four activation rows per pass, MP passes (M <= 16).  The workgroup's activations (its
// K range, all rows) and their group sums S0 sit in LDS; codes and the per-group scale /
// zero point stream through registers, D steps per batch, double-buffered.
// Requirements (else k_lowbit_mfma): 8-byte aligned rows and K ranges that fit in LDS.
// ----------------------------------------------------------------------------------
template <int BITS, int G>
struct SlotCfg {
  static constexpr int CB = BITS * G / 8;  // code bytes per row per group: 24, 16, 48, 32
  static constexpr int DW = CB / 8;        // 8-byte words per lane per step
  // steps per register batch: one (double-buffered).  Small batches keep the kernel near
  // 90-160 VGPRs (3-4 waves per SIMD), which hides more latency than deeper batches at
  // 1-2 waves per SIMD (M = 8: 20-40% faster than 96-byte batches)
  static constexpr int D = 1;
  static constexpr int SUB = G / 8;        // MFMAs per group
};

// Scale / zero-point storage: SM 0 = fp32 scales, 1 = fp16; ZM 0 = fixed offset,
// 1 = fp16 zero points, 2 = fp32.  Compile-time so that every load in the main loop is
// unconditional (addresses clamped into range, invalid data zeroed by selects) and the
// compiler can keep whole batches in flight.
template <int SM, int ZM, bool NT = true>
__device__ __forceinline__ void load_sz(const LowbitParams& p, int64_t i, float& sc, float& z) {
  if constexpr (SM == 1) sc = f16_bits_to_f32(ldw<NT>(static_cast<const uint16_t*>(p.scales) + i));
  else sc = ldw<NT>(static_cast<const float*>(p.scales) + i);
  if constexpr (ZM == 0) z = p.offset;
  else if constexpr (ZM == 1) z = f16_bits_to_f32(ldw<NT>(static_cast<const uint16_t*>(p.zeros) + i));
  else z = ldw<NT>(static_cast<const float*>(p.zeros) + i);
}

template <int BITS, int G, int MP, int SM, int ZM>
__global__ __launch_bounds__(256) void k_lowbit_slot(LowbitParams p, int gps, float* __restrict__ part) {
  using C = SlotCfg<BITS, G>;
  constexpr float OFF = BITS == 3 ? 8.f : 4.f;
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int gbeg = blockIdx.y * gps;
  const int gend = min(p.ng, gbeg + gps);
  const int GR = gend - gbeg;                 // groups in this workgroup's range
  const int GRP = (GR + 3) & ~3;              // padded S0 row
  const int KR = GR * G;                      // activations per row in range
  const int M = p.M;
  uint16_t* xs = reinterpret_cast<uint16_t*>(lds);                       // [M][KR]
  float* s0 = reinterpret_cast<float*>(lds + (((size_t)M * KR * 2 + 15) & ~(size_t)15));  // [M][GRP]

  const int col = lane & 15, slot = lane >> 4;
  const int nrow = blockIdx.x * 64 + 16 * wave + col;
  const int n = min(nrow, p.N - 1);
  const uint8_t* rowp = p.packed + (int64_t)n * p.row_bytes;
  const int64_t sidx = (int64_t)n * p.ng;
  const int steps = (GR + 3) / 4;
  const int nbatch = (steps + C::D - 1) / C::D;
  // A-operand role of this lane: row i = col, k-block = slot -> activation row mi = col >> 2
  // when col & 3 == slot
  const bool arole = (col & 3) == slot;
  const int ami = col >> 2;

  u32x2 cw[2][C::D][C::DW];
  float rs[2][C::D], rz[2][C::D];
  auto gload = [&](int b, int t0) {
#pragma unroll
    for (int d = 0; d < C::D; ++d) {
      const int g = gbeg + 4 * (t0 + d) + slot;
      const bool ok = g < gend;
      const int gc = ok ? g : gend - 1;
      const u32x2* src = reinterpret_cast<const u32x2*>(rowp + (int64_t)gc * C::CB);
#pragma unroll
      for (int w = 0; w < C::DW; ++w) cw[b][d][w] = __builtin_nontemporal_load(src + w);
      float sc, z;
      load_sz<SM, ZM>(p, sidx + gc, sc, z);
      rs[b][d] = ok ? sc : 0.f;
      rz[b][d] = OFF + z;
    }
  };
  gload(0, 0);  // the first codes are in flight while the activations are staged

  // activations of the range -> LDS (16-byte pieces); each piece's 8 values are summed and
  // the G/8 pieces of a group (consecutive lanes) combined by a fixed butterfly -> S0
  const int pieces = KR / 8;
  for (int q0 = 0; q0 < M * pieces; q0 += 256) {
    const int q = q0 + tid;
    i32x4 v = i32x4{0, 0, 0, 0};
    int m = 0, c = 0;
    if (q < M * pieces) {
      m = q / pieces;
      c = q - m * pieces;
      v = *reinterpret_cast<const i32x4*>(p.x + (int64_t)m * p.ldx + (int64_t)gbeg * G + c * 8);
      reinterpret_cast<i32x4*>(xs)[q] = v;
    }
    float t = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t dv = static_cast<uint32_t>(v[e]);
      t += bf16_bits_to_f32(dv & 0xffffu);
      t += bf16_bits_to_f32(dv >> 16);
    }
#pragma unroll
    for (int off = 1; off < G / 8; off <<= 1) t += __shfl_xor(t, off, 64);
    if (q < M * pieces && c % (G / 8) == 0) s0[m * GRP + c / (G / 8)] = t;
  }
  for (int q = tid; q < M * GRP; q += 256)
    if (q - (q / GRP) * GRP >= GR) s0[q] = 0.f;
  __syncthreads();

  f32x4 y[MP];
#pragma unroll
  for (int pp = 0; pp < MP; ++pp) y[pp] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int b, int t0) {
#pragma unroll
    for (int d = 0; d < C::D; ++d) {
      const int t = min(t0 + d, steps - 1);  // steps past the end carry zero scales
      uint32_t f[2 * C::DW + 1];
#pragma unroll
      for (int w = 0; w < C::DW; ++w) {
        f[2 * w] = cw[b][d][w].x;
        f[2 * w + 1] = cw[b][d][w].y;
      }
      f[2 * C::DW] = 0u;
      f32x4 r[MP];
#pragma unroll
      for (int pp = 0; pp < MP; ++pp) r[pp] = f32x4{0.f, 0.f, 0.f, 0.f};
      // activation block of this lane: group 4t + slot of the range (clamped; unused
      // lanes and groups are zeroed below)
      const int ga = min(4 * t + slot, GR - 1);
#pragma unroll
      for (int h = 0; h < C::SUB; ++h) {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        u32x4 bw;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int bp = BITS * (8 * h + 2 * e);
          const int wi = bp >> 5, o = bp & 31;
          uint32_t tt;
          if (o + 2 * BITS <= 32)
            tt = __builtin_amdgcn_ubfe(f[wi], o, 2 * BITS);
          else
            tt = __builtin_amdgcn_ubfe(__builtin_amdgcn_alignbit(f[wi + 1], f[wi], o), 0, 2 * BITS);
          bw[e] = pair_bf16<BITS>(tt, p.pair_mask, p.pair_base);
        }
#pragma unroll
        for (int pp = 0; pp < MP; ++pp) {
          const int m = 4 * pp + ami;
          const bool use = arole && m < M;
          const int mc = m < M ? m : 0;
          i32x4 xv = *reinterpret_cast<const i32x4*>(xs + mc * KR + ga * G + 8 * h);
          xv = use ? xv : i32x4{0, 0, 0, 0};
          r[pp] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xv),
                                                          __builtin_bit_cast(bf16x8, bw), r[pp], 0, 0, 0);
        }
      }
      // scale / zero point of groups 4t + q of this row live in lanes col + 16 q
      float sq[4], cq[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        sq[q] = __shfl(rs[b][d], col + 16 * q, 64);
        cq[q] = __shfl(rz[b][d], col + 16 * q, 64);
      }
#pragma unroll
      for (int pp = 0; pp < MP; ++pp) {
        const int m = min(4 * pp + slot, M - 1);  // D row 4*(l>>4)+q: activation row l >> 4
        const f32x4 sm = *reinterpret_cast<const f32x4*>(s0 + m * GRP + 4 * t);
#pragma unroll
        for (int q = 0; q < 4; ++q) y[pp][q] = fmaf(sq[q], fmaf(-cq[q], sm[q], r[pp][q]), y[pp][q]);
      }
    }
  };

  for (int bt = 0; bt < nbatch; bt += 2) {
    if (bt + 1 < nbatch) gload(1, (bt + 1) * C::D);
    compute(0, bt * C::D);
    if (bt + 2 < nbatch) gload(0, (bt + 2) * C::D);
    if (bt + 1 < nbatch) compute(1, (bt + 1) * C::D);
  }

  if (nrow >= p.N) return;
#pragma unroll
  for (int pp = 0; pp < MP; ++pp) {
    const int m = 4 * pp + slot;
    if (m >= M) continue;
    // lane (n, mi) holds the four group partials of row m in y[pp][0..3]: sum them in order
    const float v = add_rn(add_rn(add_rn(y[pp][0], y[pp][1]), y[pp][2]), y[pp][3]);
    if (part)
      part[((int64_t)blockIdx.y * 16 + m) * p.N + nrow] = v;
    else
      p.y[(int64_t)m * p.ldy + nrow] = v;
  }
}

// ----------------------------------------------------------------------------------
// GEMM for 3..16 bf16 activation rows in one launch (k_lowbit_gk): one workgroup per
// RT x 16 weight rows; its W waves split the groups (NGR consecutive groups each) and
// their partial results meet in a fixed-order LDS reduction.
//  * Codes, scales and zero points of the wave's groups for the workgroup's rows are read
//    as contiguous row ranges (16-byte code pieces and 4-byte scale words, 64 lanes per
//    load) and staged in the wave's LDS area.  The activations of the wave's k range go
//    to VGPRs (PF groups in flight) and serve all RT row tiles.
//  * Per group and row tile, lane l takes quarter q = l >> 4 (G/4 codes) of weight row
//    n = l & 15 and the same k range of activation row m = l & 15:
//    v_mfma_f32_16x16x32_bf16 with A = x and B = (OFF + code) pairs, G/32 MFMAs from zero,
//    so D[m][n] = R = sum_k x (OFF + c), and (int2: OFF = 0, the pairs from FP4
//    conversions of the code bytes and the activations in the matching order)
//      y[m][n] += scale * (R - (OFF + zero) * S0[m, g]),
//    S0 the group's activation sum: a second MFMA of the same A with an all-ones B, which
//    lands in the D layout (m = 4 (l >> 4) + r) and serves every row tile.
// Rows m >= M read as 0 and issue no activation loads.
// ----------------------------------------------------------------------------------
// int2 B operands come from FP4 conversions (as in k_lowbit_valu): a code byte gives the
// bf16 pairs (c0, c2) and (c1, c3).  An MFMA takes two bytes' pairs as
// (c0, c2, c1, c3, c4, c6, c5, c7), so the activations of those 8 k are arranged the same
// way: (x0,x1),(x2,x3),(x4,x5),(x6,x7) -> (x0,x2),(x1,x3),(x4,x6),(x5,x7).
__device__ __forceinline__ i32x4 fp4_pair_order(i32x4 v) {
  const uint32_t a = (uint32_t)v[0], b = (uint32_t)v[1], c = (uint32_t)v[2], d = (uint32_t)v[3];
  return i32x4{(int)__builtin_amdgcn_perm(b, a, 0x05040100u), (int)__builtin_amdgcn_perm(b, a, 0x07060302u),
               (int)__builtin_amdgcn_perm(d, c, 0x05040100u), (int)__builtin_amdgcn_perm(d, c, 0x07060302u)};
}

constexpr int kGkMaxWaves = 16;
template <int G>
constexpr int kGkGroupsShort = G == 64 ? 8 : 4;  // 2-3 row tiles, every activation in VGPRs
template <int G>
constexpr int kGkGroupsLong = G == 64 ? 12 : 6;  // one row tile, activations streamed
// int2 with G = 64 and at most 64 groups takes 4 groups per wave (16 waves): 11008 x 4096
// at M=8 9.58 -> 9.17 us; int3 keeps 8 (4: 12.9 -> 15.8 us)
template <int BITS, int G>
constexpr int kGkGroupsShortFine = BITS == 2 && G == 64 ? 4 : kGkGroupsShort<G>;
template <int G, int NGR, int RT>
// the short form (RT > 1) holds every activation of the wave in VGPRs; the long form keeps
// two groups of activations in flight: 4096 x 11008 at M=8, int2 12.4 -> 11.6 us and int3
// 13.7 -> 13.4 us against eight (twelve: 14.8 / 16.4 us)
constexpr int kGkPrefetch = RT > 1 ? NGR : 2;

template <int BITS, int G, int SM, int ZM, int NGR, int RT>
struct GkLds {
  static constexpr int CB = BITS * G / 8;
  static constexpr int RB = NGR * CB;         // code bytes per row in a wave's range
  static constexpr int RBP = RB + 16;         // 16-byte rows for ds_write_b128, 4 banks apart
  static constexpr int ES = SM == 1 ? 2 : 4;  // bytes per scale
  static constexpr int EZ = ZM == 0 ? 0 : (ZM == 1 ? 2 : 4);
  static constexpr int SWR = NGR * ES / 4;    // scale words per row (NGR even)
  static constexpr int ZWR = NGR * EZ / 4;
  static constexpr int CODE = RT * 16 * RBP;
  static constexpr int WORDS = RT * 16 * (SWR + ZWR);
  static constexpr int WAVE = CODE + 4 * WORDS;       // bytes of LDS per wave
  static_assert(WAVE >= 64 * 16 * RT, "the partials reuse the staging area");
};

template <int BITS, int G, int SM, int ZM, int NGR, int RT>
__global__ __launch_bounds__(kGkMaxWaves * 64) void k_lowbit_gk(LowbitParams p) {
  using L = GkLds<BITS, G, SM, ZM, NGR, RT>;
  constexpr float OFF = BITS == 3 ? 8.f : 0.f;
  constexpr int CB = L::CB;
  constexpr int QB = CB / 4;        // code bytes of a lane quarter
  constexpr int QC = G / 4;         // codes of a lane quarter
  constexpr int NJ = G / 32;        // MFMAs per group
  constexpr int PF = kGkPrefetch<G, NGR, RT>;
  static_assert(RT == 1 || PF == NGR, "row tiles share the wave's activations");
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  // one argument of each 64-byte argument line, requested together at entry (the compiler
  // otherwise waits for the first line before asking for the second)
  asm volatile("" ::"s"(p.x), "s"(p.M));
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int W = blockDim.x >> 6;
  const int col = lane & 15, q = lane >> 4;
  const int n0 = blockIdx.x * 16 * RT;
  const int gb = wave * NGR;
  const int M = p.M;
  const bool mval = col < M;
  const uint16_t* xr = p.x + (int64_t)min(col, M - 1) * p.ldx + q * QC;
  uint8_t* area = lds + (size_t)wave * L::WAVE;
  uint32_t* lc = reinterpret_cast<uint32_t*>(area);                     // codes [RT*16][RBP]
  uint32_t* lw = reinterpret_cast<uint32_t*>(area + L::CODE);           // scales, then zeros

  // codes: 16-byte pieces of each row's range (pieces past the row's last group read its
  // last 16 bytes again; pieces past the range are loaded but not stored)
  constexpr int PPR = L::RB / 16;
  constexpr int TOT = RT * 16 * PPR;
  constexpr int NPL = (TOT + 63) / 64;
  const int vb = p.ng * CB;
  i32x4 cp[NPL];
#pragma unroll
  for (int u = 0; u < NPL; ++u) {
    const int t = min(lane + 64 * u, TOT - 1), r = t / PPR;
    const int o = min(gb * CB + (t - r * PPR) * 16, vb - 16);
    cp[u] = *reinterpret_cast<const i32x4*>(p.packed + (int64_t)min(n0 + r, p.N - 1) * p.row_bytes + o);
  }
  // scale / zero words of each row's range (words past the row's last group repeat its
  // last word: those groups get scale 0 below)
  constexpr int SWT = RT * 16 * L::SWR, TWT = L::WORDS;
  constexpr int NWL = (TWT + 63) / 64;
  uint32_t sw[NWL];
#pragma unroll
  for (int u = 0; u < NWL; ++u) {
    const int t = min(lane + 64 * u, TWT - 1);
    const bool isz = t >= SWT;
    const int tt = isz ? t - SWT : t;
    const int wr = isz ? L::ZWR : L::SWR, eb = isz ? L::EZ : L::ES;
    const int r = tt / wr, wi = tt - r * wr;
    const int64_t row = min(n0 + r, p.N - 1);
    const int64_t rw = (int64_t)p.ng * eb / 4;  // words per row of the array
    const int64_t w = min((int64_t)gb * eb / 4 + wi, rw - 1);
    const uint32_t* src = static_cast<const uint32_t*>(isz ? p.zeros : p.scales);
    sw[u] = src[row * rw + w];
  }
  i32x4 xv[PF][NJ];
  auto xload = [&](int b, int i) {
    const int g = min(gb + i, p.ng - 1);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      i32x4 v = {0, 0, 0, 0};
      if (mval) v = *reinterpret_cast<const i32x4*>(xr + (int64_t)g * G + 8 * j);
      xv[b][j] = BITS == 2 ? fp4_pair_order(v) : v;
    }
  };
#pragma unroll
  for (int i = 0; i < PF; ++i) xload(i, i);
#pragma unroll
  for (int u = 0; u < NPL; ++u) {
    const int t = lane + 64 * u, r = t / PPR;
    if (t < TOT) *reinterpret_cast<i32x4*>(lc + (r * L::RBP + (t - r * PPR) * 16) / 4) = cp[u];
  }
#pragma unroll
  for (int u = 0; u < NWL; ++u) {
    const int t = lane + 64 * u;
    if (t < TWT) lw[t] = sw[u];
  }
  // the staging area is the wave's own: its LDS writes complete in order before its reads,
  // so no workgroup barrier (each wave starts as soon as its own codes have landed)
  __builtin_amdgcn_wave_barrier();
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

  // the lane's quarter field of group i in row tile rt: QB bytes at i * CB + q * QB of its
  // row (2- or 4-byte aligned), as a little-endian bit field
  auto field = [&](int rt, int i, uint32_t (&f)[3]) {
    const int o = (rt * 16 + col) * L::RBP + i * CB + q * QB;
    const uint32_t* w = lc + (o >> 2);
    if constexpr (QB == 6) {
      const uint32_t d0 = w[0], d1 = w[1];
      const int sh = (o & 3) * 8;
      f[0] = __builtin_amdgcn_alignbit(d1, d0, sh);
      f[1] = d1 >> sh;
      f[2] = 0;
    } else {
      f[0] = w[0];
      f[1] = QB >= 8 ? w[1] : 0u;
      f[2] = QB >= 12 ? w[2] : 0u;
    }
  };
  auto scale_zero = [&](int rt, int i, float& sc, float& cz) {
    const int e = (rt * 16 + col) * NGR + i;
    if constexpr (SM == 1) sc = f16_bits_to_f32(reinterpret_cast<const uint16_t*>(lw)[e]);
    else sc = __uint_as_float(lw[e]);
    float z;
    if constexpr (ZM == 0) z = p.offset;
    else if constexpr (ZM == 1) z = f16_bits_to_f32(reinterpret_cast<const uint16_t*>(lw + SWT)[e]);
    else z = __uint_as_float(lw[SWT + e]);
    sc = gb + i < p.ng ? sc : 0.f;
    cz = OFF + z;
  };

  const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});
  f32x4 y[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) y[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < NGR; ++i) {
    const int b = i % PF;
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xv[b][j]), ones, s0, 0, 0, 0);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      uint32_t cf[3];
      field(rt, i, cf);
      f32x4 d = {0.f, 0.f, 0.f, 0.f};
      if constexpr (BITS == 2) {
        typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
#pragma unroll
        for (int wd = 0; wd < NJ / 2; ++wd) {  // one code word = 16 codes = two MFMAs
          const uint32_t lo = cf[wd] & 0x33333333u, hi = (cf[wd] >> 2) & 0x33333333u;
          const bf16x2 pl[4] = {__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(lo, 2.f, 0),
                                __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(lo, 2.f, 1),
                                __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(lo, 2.f, 2),
                                __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(lo, 2.f, 3)};
          const bf16x2 ph[4] = {__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(hi, 2.f, 0),
                                __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(hi, 2.f, 1),
                                __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(hi, 2.f, 2),
                                __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(hi, 2.f, 3)};
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const u32x4 bw = {__builtin_bit_cast(uint32_t, pl[2 * h]), __builtin_bit_cast(uint32_t, ph[2 * h]),
                              __builtin_bit_cast(uint32_t, pl[2 * h + 1]), __builtin_bit_cast(uint32_t, ph[2 * h + 1])};
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xv[b][2 * wd + h]),
                                                        __builtin_bit_cast(bf16x8, bw), d, 0, 0, 0);
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          u32x4 bw;
#pragma unroll
          for (int e = 0; e < 4; ++e) bw[e] = code_pair<BITS>(cf, BITS * (8 * j + 2 * e), p.pair_mask, p.pair_base);
          d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xv[b][j]),
                                                      __builtin_bit_cast(bf16x8, bw), d, 0, 0, 0);
        }
      }
      float sc, cz;
      scale_zero(rt, i, sc, cz);
#pragma unroll
      for (int r = 0; r < 4; ++r) y[rt][r] = fmaf(sc, fmaf(-cz, s0[r], d[r]), y[rt][r]);
    }
    if (i + PF < NGR) xload(b, i + PF);
  }

  __syncthreads();  // every wave is done with its staging area: it now holds the partials
  f32x4* red = reinterpret_cast<f32x4*>(lds);  // [W][RT][64]
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) red[(wave * RT + rt) * 64 + lane] = y[rt];
  __syncthreads();
  // row tile rt is summed over the waves in order by wave rt % W
  for (int rt = wave; rt < RT; rt += W) {
    const int nn = n0 + rt * 16 + col;
    f32x4 t = red[rt * 64 + lane];
    for (int w = 1; w < W; ++w) t += red[(w * RT + rt) * 64 + lane];
    if (nn < p.N) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 4 * q + r;
        if (m < M) p.y[(int64_t)m * p.ldy + nn] = t[r];
      }
    }
  }
}

template <int BITS, int G, int NGR, int RT>
void launch_gk_n(const LowbitParams& p, hipStream_t s) {
  const int waves = (int)cdiv(p.ng, NGR);
  const dim3 grid((unsigned)cdiv(p.N, 16 * RT)), block(waves * 64);
  if (p.scale_f16) {
    const size_t lds = (size_t)waves * GkLds<BITS, G, 1, 1, NGR, RT>::WAVE;
    hipLaunchKernelGGL((k_lowbit_gk<BITS, G, 1, 1, NGR, RT>), grid, block, lds, s, p);
  } else {
    const size_t lds = (size_t)waves * GkLds<BITS, G, 0, 0, NGR, RT>::WAVE;
    hipLaunchKernelGGL((k_lowbit_gk<BITS, G, 0, 0, NGR, RT>), grid, block, lds, s, p);
  }
}

// the short form (two or three row tiles) while its waves fit a workgroup
template <int BITS, int G>
void launch_gk(const LowbitParams& p, hipStream_t s) {
  // int2 takes three row tiles per workgroup: 11008 rows make 230 workgroups, at most one
  // per CU (9.8 us against 10.9 us with two tiles at M=8); int3 keeps two (12.9 against 13.3)
  constexpr int RT = BITS == 2 ? 3 : 2;
  constexpr int FINE = kGkGroupsShortFine<BITS, G>;
  if (FINE != kGkGroupsShort<G> && p.ng <= kGkMaxWaves * FINE) launch_gk_n<BITS, G, FINE, RT>(p, s);
  else if (p.ng <= kGkMaxWaves * kGkGroupsShort<G>) launch_gk_n<BITS, G, kGkGroupsShort<G>, RT>(p, s);
  else launch_gk_n<BITS, G, kGkGroupsLong<G>, 1>(p, s);
}

// ----------------------------------------------------------------------------------
// Decode GEMV for M <= 2 bf16 activation rows (k_lowbit_valu): one wave per weight row,
// rows dealt round-robin to the waves of a persistent grid, the next row's codes in
// flight while the current one is reduced.  Lane l reads the LB-byte piece l + 64 j of
// the row (int3: 12 bytes = 32 codes, int2: 16 bytes = 64 codes): every wave load is one
// contiguous run of 64 * LB bytes.  Codes become bf16 (OFF + c) pairs (as for the MFMA
// kernels) and meet the activations in v_dot2_f32_bf16; per piece
//   y += scale * (R_piece - (OFF + zero) * S_piece),   S_piece = sum of x over the piece,
// which sums to the per-group formula because a piece never straddles a group.  The
// activations and the per-piece sums live in LDS, one copy per workgroup.  The activations
// are stored piece-transposed: 16-byte chunk v of piece c of row m sits at chunk
// (m * CH + v) * 64J + c (CH chunks per piece, pieces padded to 64J), so the 64 lanes of
// a wave (64 consecutive pieces) read 64 consecutive chunks -- with pieces laid end to
// end, lane strides of 64 or 128 bytes put every lane of a 16-byte read on the same few
// banks -- and each read is a per-lane base plus a constant offset.
// ----------------------------------------------------------------------------------
constexpr int kValuThreads = 512;  // 8 waves: one staged copy of x serves 8 row streams
// activation rows taken by the VALU kernel: its dot work grows with M while the unpack
// does not, and from M = 4 on the MFMA slot kernel is faster
constexpr int kValuMaxM = 2;
constexpr size_t kValuLdsMax = 144 * 1024;     // staged activations + piece sums per workgroup

template <int BITS>
struct ValuCfg {
  static constexpr int LB = BITS == 3 ? 12 : 16;  // bytes per lane piece
  static constexpr int CPL = LB * 8 / BITS;       // codes per piece: 32 / 64
  static constexpr int NW = LB / 4;               // dwords per piece
};

// int2 pieces skip the OFF + c pairs: a code word w (16 codes) gives w & 0x33333333 and
// (w >> 2) & 0x33333333, whose byte k holds codes (4k, 4k+2) and (4k+1, 4k+3) as the low
// bits of two nibbles.  Read as FP4 (e2m1) those nibbles are 0, 0.5, 1, 1.5, so
// v_cvt_scalef32_pk_bf16_fp4 with scale 2 turns each byte into an exact bf16 pair (c, c').
// The activations are staged to match: per 16-code word, a chunk of the even-indexed x and
// a chunk of the odd-indexed x.  That is 11 VALU ops per 16 codes before the dot products,
// against 24 for the multiply / bitop3 pairs.
template <int BITS, int G, int MB, int J, int SM, int ZM>
__global__ __launch_bounds__(kValuThreads) void k_lowbit_valu(LowbitParams p) {
  using C = ValuCfg<BITS>;
  constexpr float OFF = BITS == 3 ? 8.f : 0.f;
  constexpr int W = kValuThreads / 64;
  typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int K = p.K, M = p.M;
  const int npc = K / C::CPL;  // pieces per row
  uint16_t* xs = reinterpret_cast<uint16_t*>(lds);                                  // [MB][CH][PS] chunks
  constexpr int CH = C::CPL / 8;  // 16-byte activation chunks per piece
  constexpr int PS = 64 * J;      // piece stride of the transposed activations (>= npc)
  float* ps = reinterpret_cast<float*>(lds + (size_t)MB * CH * PS * 16);                   // [MB][npc]

  // wave-uniform row stream (scalar registers): rows wave_id + i * nwaves
  const int wave_id = __builtin_amdgcn_readfirstlane(blockIdx.x * W + (tid >> 6));
  const int nwaves = gridDim.x * W;
  const int ng = p.ng;
  // per-lane constants: piece j of this lane, its byte offset, scale index, LDS offsets
  int poff[J], pgrp[J], ppc[J];
  bool pval[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int pc = lane + 64 * j;
    pval[j] = pc < npc;
    const int pcc = pval[j] ? pc : npc - 1;
    poff[j] = pcc * C::LB;
    pgrp[j] = pcc * C::CPL / G;
    ppc[j] = pcc;
  }

  constexpr int R = 1;  // rows per register batch
  uint32_t cw[2][R][J][C::NW];
  float rs[2][R][J], rz[2][R][J];
  // batch bt = rows wave_id + (bt * R + i) * nwaves, i < R (rows past N load row N-1)
  auto gload = [&](int b, int bt) {
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int row = min(wave_id + (bt * R + i) * nwaves, p.N - 1);
      const uint8_t* rp = p.packed + (int64_t)row * p.row_bytes;
      const int64_t sb = (int64_t)row * ng;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        if constexpr (BITS == 3) {
          const u32x3 v = __builtin_nontemporal_load(reinterpret_cast<const u32x3*>(rp + poff[j]));
          cw[b][i][j][0] = v.x;
          cw[b][i][j][1] = v.y;
          cw[b][i][j][2] = v.z;
        } else {
          const i32x4 v = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(rp + poff[j]));
#pragma unroll
          for (int w = 0; w < 4; ++w) cw[b][i][j][w] = static_cast<uint32_t>(v[w]);
        }
        float sc, z;
        load_sz<SM, ZM>(p, sb + pgrp[j], sc, z);
        rs[b][i][j] = pval[j] ? sc : 0.f;
        rz[b][i][j] = OFF + z;
      }
    }
  };
  const int nrows = wave_id < p.N ? (p.N - 1 - wave_id) / nwaves + 1 : 0;  // rows of this wave
  const int nbt = (nrows + R - 1) / R;
  // the first kXRegs activation chunks per thread are requested before the codes, so the
  // staging below waits for them only, not for the codes in flight behind them (loads
  // return in order).  Short rows hold one staging unit: int2 11008 x 4096 went 6.97 ->
  // 6.58 us at M = 1 and 8.70 -> 8.12 us at M = 2 over staging after the codes.
  constexpr int kXRegs = J >= 3 ? 6 : 2;
  // staging unit: one 16-byte chunk (int3) or one 16-code word's 32 bytes (int2)
  constexpr int U = BITS == 2 ? 2 : 1;
  constexpr int kXU = kXRegs / U;
  const int upr = K / (8 * U);  // units per activation row
  const int xu = M * upr;
  auto uload = [&](int q, i32x4* v) {
    const int m = q / upr, c = q - m * upr;
#pragma unroll
    for (int h = 0; h < U; ++h)
      v[h] = *reinterpret_cast<const i32x4*>(p.x + (int64_t)m * p.ldx + (int64_t)(c * U + h) * 8);
  };
  auto ustore = [&](int q, const i32x4* v) {
    const int m = q / upr, c = q - m * upr;
    i32x4* xc = reinterpret_cast<i32x4*>(xs);
    if constexpr (U == 1) {
      xc[(m * CH + c % CH) * PS + c / CH] = v[0];
    } else {
      // word w of piece pc: even-indexed x -> chunk 2w, odd-indexed x -> chunk 2w + 1
      const int pc = c / 4, w = c % 4;
      i32x4 ev, od;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t a = static_cast<uint32_t>(v[k / 2][(2 * k) % 4]);
        const uint32_t b2 = static_cast<uint32_t>(v[k / 2][(2 * k + 1) % 4]);
        ev[k] = static_cast<int>(__builtin_amdgcn_perm(b2, a, 0x05040100u));
        od[k] = static_cast<int>(__builtin_amdgcn_perm(b2, a, 0x07060302u));
      }
      xc[(m * CH + 2 * w) * PS + pc] = ev;
      xc[(m * CH + 2 * w + 1) * PS + pc] = od;
    }
  };
  i32x4 xr[kXU > 0 ? kXU : 1][U];
#pragma unroll
  for (int i = 0; i < kXU; ++i) {
    const int q = tid + i * kValuThreads;
    uload(q < xu ? q : 0, xr[i]);
  }
  if (nbt > 0) gload(0, 0);  // the first rows' codes are in flight during the staging

  // activations -> LDS, per-piece sums -> LDS
#pragma unroll
  for (int i = 0; i < kXU; ++i) {
    const int q = tid + i * kValuThreads;
    if (q < xu) ustore(q, xr[i]);
  }
  for (int q = tid + kXU * kValuThreads; q < xu; q += kValuThreads) {
    i32x4 v[U];
    uload(q, v);
    ustore(q, v);
  }
  __syncthreads();
  for (int q = tid; q < M * npc; q += kValuThreads) {
    const int m = q / npc, c = q - (q / npc) * npc;
    const i32x4* xp = reinterpret_cast<const i32x4*>(xs) + m * CH * PS + c;
    float t = 0.f;
    for (int v = 0; v < CH; ++v) {
      const i32x4 d = xp[v * PS];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        t += bf16_bits_to_f32(static_cast<uint32_t>(d[e]) & 0xffffu);
        t += bf16_bits_to_f32(static_cast<uint32_t>(d[e]) >> 16);
      }
    }
    ps[q] = t;
  }
  __syncthreads();

  auto compute = [&](int b, int bt) {
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int row = wave_id + (bt * R + i) * nwaves;
      if (row >= p.N) break;
      float acc[MB];
#pragma unroll
      for (int m = 0; m < MB; ++m) acc[m] = 0.f;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        float r[MB];
#pragma unroll
        for (int m = 0; m < MB; ++m) r[m] = 0.f;
        if constexpr (BITS == 2) {
#pragma unroll
          for (int w = 0; w < C::NW; ++w) {  // 16 codes per word: 8 bf16 pairs
            const uint32_t lo = cw[b][i][j][w] & 0x33333333u;
            const uint32_t hi = (cw[b][i][j][w] >> 2) & 0x33333333u;
            const bf16x2 pl[4] = {__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(lo, 2.f, 0),
                                  __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(lo, 2.f, 1),
                                  __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(lo, 2.f, 2),
                                  __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(lo, 2.f, 3)};
            const bf16x2 ph[4] = {__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(hi, 2.f, 0),
                                  __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(hi, 2.f, 1),
                                  __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(hi, 2.f, 2),
                                  __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(hi, 2.f, 3)};
#pragma unroll
            for (int m = 0; m < MB; ++m) {
              if (m < M) {
                const i32x4* xc = reinterpret_cast<const i32x4*>(xs) + (m * CH + 2 * w) * PS + ppc[j];
                const i32x4 xe = xc[0], xo = xc[PS];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                  const uint32_t e0 = static_cast<uint32_t>(xe[k]), o0 = static_cast<uint32_t>(xo[k]);
                  r[m] = __builtin_amdgcn_fdot2_f32_bf16(pl[k], __builtin_bit_cast(bf16x2, e0), r[m], false);
                  r[m] = __builtin_amdgcn_fdot2_f32_bf16(ph[k], __builtin_bit_cast(bf16x2, o0), r[m], false);
                }
              }
            }
          }
        } else
#pragma unroll
        for (int v = 0; v < C::CPL / 8; ++v) {  // 8 codes per step: 4 bf16 pairs
          uint32_t bw[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int bp = BITS * (8 * v + 2 * e);
            const int wi = bp >> 5, o = bp & 31;
            uint32_t tt;
            if (o + 2 * BITS <= 32 || wi + 1 >= C::NW)
              tt = __builtin_amdgcn_ubfe(cw[b][i][j][wi], o, 2 * BITS);
            else
              tt = __builtin_amdgcn_ubfe(__builtin_amdgcn_alignbit(cw[b][i][j][wi + 1], cw[b][i][j][wi], o), 0, 2 * BITS);
            bw[e] = pair_bf16<BITS>(tt, p.pair_mask, p.pair_base);
          }
#pragma unroll
          for (int m = 0; m < MB; ++m) {
            if (m < M) {
              const i32x4 xv = reinterpret_cast<const i32x4*>(xs)[(m * CH + v) * PS + ppc[j]];
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                // copy the element out first: bit-casting a vector element expression reads
                // element 0 of the whole vector with this compiler
                const uint32_t xe = static_cast<uint32_t>(xv[e]);
                r[m] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, bw[e]),
                                                       __builtin_bit_cast(bf16x2, xe), r[m], false);
              }
            }
          }
        }
#pragma unroll
        for (int m = 0; m < MB; ++m)
          if (m < M) acc[m] = fmaf(rs[b][i][j], fmaf(-rz[b][i][j], ps[m * npc + ppc[j]], r[m]), acc[m]);
      }
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        const float v = wave_sum_dpp(acc[m]);
        if (lane == 0 && m < M) p.y[(int64_t)m * p.ldy + row] = v;
      }
    }
  };

  for (int bt = 0; bt < nbt; bt += 2) {
    if (bt + 1 < nbt) gload(1, bt + 1);
    compute(0, bt);
    if (bt + 2 < nbt) gload(0, bt + 2);
    if (bt + 1 < nbt) compute(1, bt + 1);
  }
}

// y[m, n] = sum over t < rpx (activation split terms), then over splits s, of
// part[s][rpx*m + t][n] -- fixed order.
__global__ __launch_bounds__(256) void k_lowbit_reduce(const float* __restrict__ part, int S, int rpx,
                                                       int M, int N, float* __restrict__ y, int64_t ldy) {
  const int64_t i = blockIdx.x * 256ll + threadIdx.x;
  if (i >= (int64_t)M * N) return;
  const int64_t m = i / N, n = i - m * N;
  float acc = 0.f;
  for (int t = 0; t < rpx; ++t) {
    float v = 0.f;
    for (int s = 0; s < S; ++s) v = add_rn(v, part[((int64_t)s * 16 + rpx * m + t) * N + n]);
    acc = t == 0 ? v : add_rn(acc, v);
  }
  y[m * ldy + n] = acc;
}

// x (f32 or bf16) -> bf16 activation rows: bf16 x is copied; fp32 row m becomes rows
// 3m, 3m+1, 3m+2 = h, bf16(x - h), bf16(x - h - m) (an exact three-term split).
__global__ __launch_bounds__(256) void k_lowbit_prep(const void* __restrict__ x, int x_dtype,
                                                     int64_t ldx, int M, int K,
                                                     uint16_t* __restrict__ xb) {
  const int64_t i = blockIdx.x * 256ll + threadIdx.x;
  if (i >= (int64_t)M * K) return;
  const int64_t m = i / K, k = i - m * K;
  if (x_dtype == QS_BF16) {
    xb[m * K + k] = static_cast<const uint16_t*>(x)[m * ldx + k];
  } else {
    const float v = static_cast<const float*>(x)[m * ldx + k];
    const uint16_t h = f32_to_bf16_bits(v);
    const float r1 = v - bf16_bits_to_f32(h);
    const uint16_t md = f32_to_bf16_bits(r1);
    const float r2 = r1 - bf16_bits_to_f32(md);
    xb[(3 * m) * K + k] = h;
    xb[(3 * m + 1) * K + k] = md;
    xb[(3 * m + 2) * K + k] = f32_to_bf16_bits(r2);
  }
}

// S0[m, g] = sum of the G bf16 activations of group g, fixed order.  One wave per (m, g).
__global__ __launch_bounds__(256) void k_group_sums(const uint16_t* __restrict__ xb, int M, int K,
                                                    int G, float* __restrict__ s0) {
  const int lane = threadIdx.x & 63;
  const int64_t w = blockIdx.x * 4ll + (threadIdx.x >> 6);
  const int ng = K / G;
  if (w >= (int64_t)M * ng) return;
  const int64_t m = w / ng, g = w - m * ng;
  float v = 0.f;
  for (int k = lane; k < G; k += 64) v += bf16_bits_to_f32(xb[m * K + g * G + k]);
  v = wave_sum(v);
  if (lane == 0) s0[w] = v;
}

// y[m, n] = y3[3m, n] + y3[3m+1, n] + y3[3m+2, n]
__global__ __launch_bounds__(256) void k_lowbit_combine(const float* __restrict__ y3, int M, int N,
                                                        float* __restrict__ y, int64_t ldy) {
  const int64_t i = blockIdx.x * 256ll + threadIdx.x;
  if (i >= (int64_t)M * N) return;
  const int64_t m = i / N, n = i - m * N;
  y[m * ldy + n] = add_rn(add_rn(y3[(3 * m) * N + n], y3[(3 * m + 1) * N + n]), y3[(3 * m + 2) * N + n]);
}

// w[n, k] = (float(code) - zero) * scale, fp32 (reference _dequant_int3/_int2 order).
__global__ __launch_bounds__(256) void k_lowbit_dequant(LowbitParams p, int bits, int G, float* __restrict__ out) {
  const int64_t i = blockIdx.x * 256ll + threadIdx.x;
  if (i >= (int64_t)p.N * p.K) return;
  const int64_t n = i / p.K, k = i - n * p.K;
  const int64_t bit = k * bits;
  const uint8_t* row = p.packed + n * p.row_bytes;
  uint32_t v = row[bit >> 3] >> (bit & 7);
  if ((bit & 7) + bits > 8) v |= (uint32_t)row[(bit >> 3) + 1] << (8 - (bit & 7));
  const uint32_t code = v & ((1u << bits) - 1);
  const int64_t si = n * p.ng + k / G;
  const float sc = p.scale_f16 ? f16_bits_to_f32(static_cast<const uint16_t*>(p.scales)[si])
                               : static_cast<const float*>(p.scales)[si];
  float z = p.offset;
  if (p.zeros)
    z = p.zero_f16 ? f16_bits_to_f32(static_cast<const uint16_t*>(p.zeros)[si])
                   : static_cast<const float*>(p.zeros)[si];
  out[i] = mul_rn(static_cast<float>(code) - z, sc);
}

// k_lowbit_dequant for K and the group size multiples of 4: a thread expands 4 codes of a
// row (one byte at 2 bits; 12 or 16 bits from two bytes at 3 or 4) into one 16-byte store,
// so a wave's store instruction writes 1 KB of consecutive output.  Same values; 11008 x
// 4096 fp32 out, same box: int3 140.4 -> 43.8 us, int2 124.8 -> 38.1 us against one code
// per thread.  Each thread takes U such pieces, 256 apart, with all their loads issued
// before the first store (a load behind a store would also wait for the store).
constexpr int kLowbitDequantPieces = 4;

template <int U>
__global__ __launch_bounds__(256) void k_lowbit_dequant4(LowbitParams p, int bits, int G, float* __restrict__ out) {
  const int64_t k4 = p.K / 4;
  const int64_t total = (int64_t)p.N * k4;
  // Workgroup b runs on XCD b % 8.  A row's workgroups share the row's scale and zero
  // lines, so consecutive logical indices go to one XCD and its L2 serves the repeats
  // (with the plain order the 128-byte scale line of a 4096-column row was fetched from
  // HBM by four XCDs): the first 8 * floor(grid / 8) workgroups are dealt out XCD-major.
  const int64_t nb = gridDim.x, per = nb / 8;
  const int64_t b = blockIdx.x;
  const int64_t lb = b < 8 * per ? (b % 8) * per + b / 8 : b;
  const int64_t base = lb * 256 * U;
  // the chunk's first row from one division, each piece's from a 32-bit one
  const int64_t n0 = base / k4;
  const uint32_t c0 = (uint32_t)(base - n0 * k4);
  const uint32_t mask = (1u << bits) - 1;
  uint32_t v[U];
  float sc[U], z[U];
  int64_t n[U];
  uint32_t c[U];
  bool ok[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t off = c0 + (uint32_t)(u * 256 + threadIdx.x);  // < k4 + 256 U
    const uint32_t q = off / (uint32_t)k4;
    ok[u] = base + u * 256 + threadIdx.x < total;
    n[u] = ok[u] ? n0 + q : 0;
    c[u] = ok[u] ? off - q * (uint32_t)k4 : 0u;
    const int64_t bit = (int64_t)c[u] * 4 * bits;  // 8c, 12c or 16c: the piece ends inside the row
    const uint8_t* row = p.packed + n[u] * p.row_bytes;
    v[u] = row[bit >> 3];
    if (bits > 2) v[u] |= static_cast<uint32_t>(row[(bit >> 3) + 1]) << 8;
    v[u] >>= (bit & 7);
    const int64_t si = n[u] * p.ng + (4 * (int64_t)c[u]) / G;
    sc[u] = p.scale_f16 ? f16_bits_to_f32(static_cast<const uint16_t*>(p.scales)[si])
                        : static_cast<const float*>(p.scales)[si];
    z[u] = p.offset;
    if (p.zeros)
      z[u] = p.zero_f16 ? f16_bits_to_f32(static_cast<const uint16_t*>(p.zeros)[si])
                        : static_cast<const float*>(p.zeros)[si];
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (!ok[u]) continue;
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = mul_rn(static_cast<float>((v[u] >> (bits * e)) & mask) - z[u], sc[u]);
    *reinterpret_cast<f32x4*>(out + n[u] * p.K + 4 * (int64_t)c[u]) = o;
  }
}

// Any layout the tiled kernels refuse (a group size other than 64 / 128, K not a multiple
// of the group size -- a short last group --, rows not 4-byte aligned): one wave per weight
// row, at most kAnyRows activation rows per launch.  Each lane decodes its codes like
// k_lowbit_dequant, multiplies them into its fp32 partial sums in k order, and a wave sum
// finishes each row.  A correctness path: the reference runs these stores on the CPU.
constexpr int kAnyRows = 8;

template <int XT>
__global__ __launch_bounds__(256) void k_lowbit_any(LowbitParams p, int bits, int G, const void* __restrict__ x,
                                                    int64_t ldx) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= p.N) return;
  float acc[kAnyRows];
#pragma unroll
  for (int m = 0; m < kAnyRows; ++m) acc[m] = 0.f;
  const uint8_t* row = p.packed + n * p.row_bytes;
  for (int64_t k = lane; k < p.K; k += 64) {
    const int64_t bit = k * bits;
    uint32_t v = row[bit >> 3] >> (bit & 7);
    if ((bit & 7) + bits > 8) v |= (uint32_t)row[(bit >> 3) + 1] << (8 - (bit & 7));
    const uint32_t code = v & ((1u << bits) - 1);
    const int64_t si = n * p.ng + k / G;
    const float sc = p.scale_f16 ? f16_bits_to_f32(static_cast<const uint16_t*>(p.scales)[si])
                                 : static_cast<const float*>(p.scales)[si];
    float z = p.offset;
    if (p.zeros)
      z = p.zero_f16 ? f16_bits_to_f32(static_cast<const uint16_t*>(p.zeros)[si])
                     : static_cast<const float*>(p.zeros)[si];
    const float w = mul_rn(static_cast<float>(code) - z, sc);
#pragma unroll
    for (int m = 0; m < kAnyRows; ++m) {
      if (m < p.M) {
        float xv;
        if constexpr (XT == QS_F32) xv = static_cast<const float*>(x)[m * ldx + k];
        else xv = bf16_bits_to_f32(static_cast<const uint16_t*>(x)[m * ldx + k]);
        acc[m] = fmaf(xv, w, acc[m]);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < kAnyRows; ++m) {
    if (m < p.M) {
      const float t = wave_sum(acc[m]);
      if (lane == 0) p.y[m * p.ldy + n] = t;
    }
  }
}

namespace {
constexpr size_t kSlotLds = 64 * 1024;  // activations + group sums of one workgroup's K range

template <int BITS, int G, int SM, int ZM>
void launch_slot_sz(int mp, dim3 grid, size_t lds, hipStream_t s, const LowbitParams& p, int gps, float* part) {
  if (mp == 1) hipLaunchKernelGGL((k_lowbit_slot<BITS, G, 1, SM, ZM>), grid, dim3(256), lds, s, p, gps, part);
  else if (mp == 2) hipLaunchKernelGGL((k_lowbit_slot<BITS, G, 2, SM, ZM>), grid, dim3(256), lds, s, p, gps, part);
  else if (mp == 3) hipLaunchKernelGGL((k_lowbit_slot<BITS, G, 3, SM, ZM>), grid, dim3(256), lds, s, p, gps, part);
  else hipLaunchKernelGGL((k_lowbit_slot<BITS, G, 4, SM, ZM>), grid, dim3(256), lds, s, p, gps, part);
}

// Two storage layouts get the slotted kernel: fp16 scale + fp16 zero point (the
// asymmetric G64 variant) and fp32 scales with the fixed offset (the reference layout).
template <int BITS, int G>
void launch_slot(int mp, dim3 grid, size_t lds, hipStream_t s, const LowbitParams& p, int gps, float* part) {
  if (p.scale_f16) launch_slot_sz<BITS, G, 1, 1>(mp, grid, lds, s, p, gps, part);
  else launch_slot_sz<BITS, G, 0, 0>(mp, grid, lds, s, p, gps, part);
}

template <int BITS, int G, int MB, int J>
void launch_valu_j(unsigned grid, size_t lds, hipStream_t s, const LowbitParams& p) {
  if (p.scale_f16) hipLaunchKernelGGL((k_lowbit_valu<BITS, G, MB, J, 1, 1>), dim3(grid), dim3(kValuThreads), lds, s, p);
  else hipLaunchKernelGGL((k_lowbit_valu<BITS, G, MB, J, 0, 0>), dim3(grid), dim3(kValuThreads), lds, s, p);
}

template <int BITS, int G, int MB>
void launch_valu_mb(int J, unsigned grid, size_t lds, hipStream_t s, const LowbitParams& p) {
  if (J == 1) launch_valu_j<BITS, G, MB, 1>(grid, lds, s, p);
  else if (J == 2) launch_valu_j<BITS, G, MB, 2>(grid, lds, s, p);
  else if (J == 3) launch_valu_j<BITS, G, MB, 3>(grid, lds, s, p);
  else if (J == 4) launch_valu_j<BITS, G, MB, 4>(grid, lds, s, p);
  else launch_valu_j<BITS, G, MB, 6>(grid, lds, s, p);
}

// MB: activation rows per launch (1 or 2; p.M <= MB)
template <int BITS>
void launch_valu(int J, int MB, int G, unsigned grid, size_t lds, hipStream_t s, const LowbitParams& p) {
  if (G == 64) {
    if (MB == 1) launch_valu_mb<BITS, 64, 1>(J, grid, lds, s, p);
    else launch_valu_mb<BITS, 64, 2>(J, grid, lds, s, p);
  } else {
    if (MB == 1) launch_valu_mb<BITS, 128, 1>(J, grid, lds, s, p);
    else launch_valu_mb<BITS, 128, 2>(J, grid, lds, s, p);
  }
}

template <int BITS, int G>
void launch_lowbit(const LowbitParams& p, hipStream_t s) {
  const dim3 grid((unsigned)cdiv(p.N, 16));
  if (p.ng >= 64)
    hipLaunchKernelGGL((k_lowbit_mfma<BITS, G, 8>), grid, dim3(8 * 64), 0, s, p);
  else
    hipLaunchKernelGGL((k_lowbit_mfma<BITS, G, 4>), grid, dim3(4 * 64), 0, s, p);
}

int check_lowbit(const void* packed, int64_t row_bytes, const void* scales, int bits, int G,
                 int64_t N, int64_t K) {
  if (!packed || !scales) return fail(QS_ERR_INVALID, "lowbit: null pointer");
  if (bits != 2 && bits != 3) return fail(QS_ERR_UNSUPPORTED, "lowbit: bits must be 2 or 3");
  if (G <= 0 || N <= 0 || K <= 0 || N > INT_MAX || K > INT_MAX) return fail(QS_ERR_INVALID, "lowbit: bad shape");
  if (row_bytes < (K * bits + 7) / 8) return fail(QS_ERR_INVALID, "lowbit: row_bytes too small");
  return QS_OK;
}

// the tiled kernels' layout: G 64 or 128, whole groups, 4-byte aligned rows
bool tiled_layout(const void* packed, int64_t row_bytes, int G, int64_t K) {
  return (G == 64 || G == 128) && K % G == 0 && row_bytes % 4 == 0 && aligned(packed, 4);
}
}  // namespace
}  // namespace qs

using namespace qs;

static constexpr int kLowbitMaxSplit = 8;  // K splits of k_lowbit_slot (partial-sum planes)

extern "C" int qs_lowbit_gemv(const void* x, int x_dtype, int64_t ldx, const uint8_t* packed,
                              int64_t row_bytes, const void* scales, int scale_dtype,
                              const void* zeros, int zero_dtype, float offset, int bits,
                              int group_size, float* y, int64_t ldy, int64_t M, int64_t N,
                              int64_t K, void* workspace, size_t workspace_bytes, void* stream) {
  int st = check_lowbit(packed, row_bytes, scales, bits, group_size, N, K);
  if (st) return st;
  if (!x || !y) return fail(QS_ERR_INVALID, "lowbit_gemv: null pointer");
  if (x_dtype != QS_BF16 && x_dtype != QS_F32) return fail(QS_ERR_INVALID, "lowbit_gemv: x must be BF16 or F32");
  if (scale_dtype != QS_F32 && scale_dtype != QS_F16) return fail(QS_ERR_INVALID, "lowbit_gemv: scales F32 or F16");
  if (zeros && zero_dtype != QS_F32 && zero_dtype != QS_F16) return fail(QS_ERR_INVALID, "lowbit_gemv: zeros F32 or F16");
  if (M < 0 || ldx < K || ldy < N) return fail(QS_ERR_INVALID, "lowbit_gemv: bad leading dimension");
  if (M == 0) return QS_OK;
  if (!tiled_layout(packed, row_bytes, group_size, K)) {
    LowbitParams p{};
    p.packed = packed;
    p.row_bytes = row_bytes;
    p.scales = scales;
    p.zeros = zeros;
    p.scale_f16 = scale_dtype == QS_F16;
    p.zero_f16 = zero_dtype == QS_F16;
    p.offset = offset;
    p.ldy = ldy;
    p.N = (int)N;
    p.K = (int)K;
    p.ng = (int)cdiv(K, group_size);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const size_t xe = x_dtype == QS_F32 ? 4 : 2;
    for (int64_t m0 = 0; m0 < M; m0 += kAnyRows) {
      p.M = (int)(M - m0 < kAnyRows ? M - m0 : kAnyRows);
      p.y = y + m0 * ldy;
      const void* xm = static_cast<const char*>(x) + m0 * ldx * xe;
      if (x_dtype == QS_F32)
        hipLaunchKernelGGL(k_lowbit_any<QS_F32>, dim3((unsigned)cdiv(N, 4)), dim3(256), 0, s, p, bits, group_size, xm, ldx);
      else
        hipLaunchKernelGGL(k_lowbit_any<QS_BF16>, dim3((unsigned)cdiv(N, 4)), dim3(256), 0, s, p, bits, group_size, xm, ldx);
    }
    return hip_check(hipGetLastError(), "k_lowbit_any launch");
  }
  const int rows_per_x = x_dtype == QS_F32 ? 3 : 1;
  const int mb = x_dtype == QS_F32 ? 5 : 16;  // activation rows per MFMA tile
  const int ng = (int)(K / group_size);
  const size_t need = qs_lowbit_workspace_bytes(x_dtype, M, N, K, group_size);
  if (!workspace || workspace_bytes < need)
    return fail(QS_ERR_INVALID, "lowbit_gemv: workspace of %zu bytes required", need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int cb = bits * group_size / 8;
  (void)cb;
  const bool tiled = row_bytes % 8 == 0 && aligned(packed, 8) && aligned(workspace, 16);
  // workspace: bf16 rows [16, K] | s0 [16, ng] | partial sums [kLowbitMaxSplit, 16, N]
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint16_t* xb = reinterpret_cast<uint16_t*>(ws);
  const size_t xb_bytes = ((size_t)16 * K * 2 + 255) / 256 * 256;
  float* s0 = reinterpret_cast<float*>(ws + xb_bytes);
  const size_t s0_bytes = ((size_t)16 * ng * 4 + 255) / 256 * 256;
  float* y3 = reinterpret_cast<float*>(ws + xb_bytes + s0_bytes);
  {
    // decode: M <= 2 bf16 rows, one wave per weight row
    const int cpl = bits == 3 ? 32 : 64;
    const int J = (int)cdiv(cdiv(K, cpl), 64);
    // activation rows per launch: the next power of two >= M, halved until x and the piece
    // sums fit the LDS budget; larger M runs as several launches
    auto lds_for = [&](int mbx) {  // transposed activations (pieces padded to 64 J) + piece sums
      return (size_t)mbx * J * 64 * cpl * 2 + (size_t)mbx * (K / cpl) * 4;
    };
    int mbv = M <= 1 ? 1 : 2;
    while (mbv > 1 && lds_for(mbv) > kValuLdsMax) mbv /= 2;
    const size_t lds = lds_for(mbv);
    const bool layout = (scale_dtype == QS_F16 && zeros && zero_dtype == QS_F16) || (scale_dtype == QS_F32 && !zeros);
    const int lb = bits == 3 ? 12 : 16;
    if (x_dtype == QS_BF16 && M <= kValuMaxM && layout && K % cpl == 0 && group_size % cpl == 0 && J <= 6 &&
        J != 5 && row_bytes % lb == 0 && aligned(packed, 16) && aligned(x, 16) && ldx % 8 == 0 &&
        lds <= kValuLdsMax) {
      LowbitParams p{};
      p.x = static_cast<const uint16_t*>(x);
      p.ldx = ldx;
      p.packed = packed;
      p.row_bytes = row_bytes;
      p.scales = scales;
      p.zeros = zeros;
      p.scale_f16 = scale_dtype == QS_F16;
      p.zero_f16 = zero_dtype == QS_F16;
      p.offset = offset;
      p.y = y;
      p.ldy = ldy;
      p.M = (int)M;
      p.N = (int)N;
      p.K = (int)K;
      p.ng = ng;
      pair_consts(p, bits);
      const int64_t wpb = kValuThreads / 64;
      const unsigned grid = (unsigned)(cdiv(N, wpb) < 1024 ? cdiv(N, wpb) : 1024);
      for (int64_t m0 = 0; m0 < M; m0 += mbv) {
        LowbitParams q = p;
        q.M = (int)(M - m0 < mbv ? M - m0 : mbv);
        q.x = p.x + m0 * ldx;
        q.y = p.y + m0 * ldy;
        if (bits == 3) launch_valu<3>(J, mbv, group_size, grid, lds, s, q);
        else launch_valu<2>(J, mbv, group_size, grid, lds, s, q);
      }
      return hip_check(hipGetLastError(), "k_lowbit_valu launch");
    }
  }
  {
    // 3..16 bf16 rows (and any bf16 M in chunks of 16): the single-launch group-MFMA kernel
    const bool layout = (scale_dtype == QS_F16 && zeros && zero_dtype == QS_F16) || (scale_dtype == QS_F32 && !zeros);
    const int ngr = group_size == 64 ? kGkGroupsLong<64> : kGkGroupsLong<128>;
    const int waves = (int)cdiv(ng, ngr);  // the long form's count bounds both
    const int64_t vb = K * bits / 8;  // code bytes of a row (the kernel reads 16-byte pieces)
    // scale / zero rows are read as 4-byte words: fp16 arrays need an even group count
    const bool words = aligned(scales, 4) && (!zeros || aligned(zeros, 4)) && (scale_dtype == QS_F32 || ng % 2 == 0);
    if (x_dtype == QS_BF16 && layout && words && waves <= kGkMaxWaves && aligned(x, 16) && ldx % 8 == 0 &&
        vb % 16 == 0 && row_bytes % 16 == 0 && aligned(packed, 16)) {
      LowbitParams p{};
      p.ldx = ldx;
      p.packed = packed;
      p.row_bytes = row_bytes;
      p.scales = scales;
      p.zeros = zeros;
      p.scale_f16 = scale_dtype == QS_F16;
      p.zero_f16 = zero_dtype == QS_F16;
      p.offset = offset;
      p.ldy = ldy;
      p.N = (int)N;
      p.K = (int)K;
      p.ng = ng;
      pair_consts(p, bits);
      for (int64_t m0 = 0; m0 < M; m0 += 16) {
        p.x = static_cast<const uint16_t*>(x) + m0 * ldx;
        p.y = y + m0 * ldy;
        p.M = (int)(M - m0 < 16 ? M - m0 : 16);
        if (bits == 3 && group_size == 64) launch_gk<3, 64>(p, s);
        else if (bits == 3) launch_gk<3, 128>(p, s);
        else if (group_size == 64) launch_gk<2, 64>(p, s);
        else launch_gk<2, 128>(p, s);
      }
      return hip_check(hipGetLastError(), "k_lowbit_gk launch");
    }
  }
  for (int64_t m0 = 0; m0 < M; m0 += mb) {
    const int mm = (int)((M - m0) < mb ? (M - m0) : mb);
    const int rows = mm * rows_per_x;
    const void* xm = static_cast<const char*>(x) + m0 * ldx * (x_dtype == QS_F32 ? 4 : 2);
    // slotted kernel: K split so that each workgroup's activations + group sums fit in LDS
    const int tiles = (int)cdiv(N, 64);
    int S = (int)cdiv(512, tiles);
    S = S < 1 ? 1 : (S > kLowbitMaxSplit ? kLowbitMaxSplit : S);
    int gps = (int)cdiv(ng, S);
    auto lds_of = [&](int g) {
      return (((size_t)rows * g * group_size * 2 + 15) & ~(size_t)15) + (size_t)rows * ((g + 3) & ~3) * 4;
    };
    while (lds_of(gps) > kSlotLds && S < kLowbitMaxSplit) gps = (int)cdiv(ng, ++S);
    S = (int)cdiv(ng, gps);
    const bool slot_layout = (scale_dtype == QS_F16 && zeros && zero_dtype == QS_F16) ||
                             (scale_dtype == QS_F32 && !zeros);
    const bool slot = tiled && slot_layout && lds_of(gps) <= kSlotLds;
    // bf16 activations that are 16-byte aligned feed the slotted kernel directly
    const bool x_direct = slot && x_dtype == QS_BF16 && aligned(xm, 16) && ldx % 8 == 0;
    if (!x_direct)
      hipLaunchKernelGGL(k_lowbit_prep, dim3((unsigned)cdiv((int64_t)mm * K, 256)), dim3(256), 0, s, xm, x_dtype, ldx, mm, (int)K, xb);
    if (!slot)
      hipLaunchKernelGGL(k_group_sums, dim3((unsigned)cdiv((int64_t)rows * ng, 4)), dim3(256), 0, s, xb, rows, (int)K, group_size, s0);
    LowbitParams p{};
    p.x = x_direct ? static_cast<const uint16_t*>(xm) : xb;
    p.ldx = x_direct ? ldx : K;
    p.s0 = s0;
    p.packed = packed;
    p.row_bytes = row_bytes;
    p.scales = scales;
    p.zeros = zeros;
    p.scale_f16 = scale_dtype == QS_F16;
    p.zero_f16 = zero_dtype == QS_F16;
    p.offset = offset;
    p.M = rows;
    p.N = (int)N;
    p.K = (int)K;
    p.ng = ng;
    pair_consts(p, bits);
    if (slot) {
      const bool direct = S == 1 && x_dtype == QS_BF16;
      p.y = y + m0 * ldy;
      p.ldy = ldy;
      float* part = direct ? nullptr : y3;
      const dim3 grid((unsigned)tiles, (unsigned)S);
      const int mp = (rows + 3) / 4;
      const size_t lds = lds_of(gps);
      if (bits == 3 && group_size == 64) launch_slot<3, 64>(mp, grid, lds, s, p, gps, part);
      else if (bits == 3) launch_slot<3, 128>(mp, grid, lds, s, p, gps, part);
      else if (group_size == 64) launch_slot<2, 64>(mp, grid, lds, s, p, gps, part);
      else launch_slot<2, 128>(mp, grid, lds, s, p, gps, part);
      if (!direct)
        hipLaunchKernelGGL(k_lowbit_reduce, dim3((unsigned)cdiv((int64_t)mm * N, 256)), dim3(256), 0, s, y3, S,
                           rows_per_x, mm, (int)N, y + m0 * ldy, ldy);
      continue;
    }
    if (x_dtype == QS_BF16) {
      p.y = y + m0 * ldy;
      p.ldy = ldy;
    } else {
      p.y = y3;
      p.ldy = N;
    }
    if (bits == 3 && group_size == 64) launch_lowbit<3, 64>(p, s);
    else if (bits == 3) launch_lowbit<3, 128>(p, s);
    else if (group_size == 64) launch_lowbit<2, 64>(p, s);
    else launch_lowbit<2, 128>(p, s);
    if (x_dtype == QS_F32)
      hipLaunchKernelGGL(k_lowbit_combine, dim3((unsigned)cdiv((int64_t)mm * N, 256)), dim3(256), 0, s, y3, mm, (int)N, y + m0 * ldy, ldy);
  }
  return hip_check(hipGetLastError(), "k_lowbit launch");
}

extern "C" size_t qs_lowbit_workspace_bytes(int x_dtype, int64_t M, int64_t N, int64_t K, int group_size) {
  (void)M;
  (void)x_dtype;
  const int64_t ng = group_size > 0 ? K / group_size : 0;
  const size_t xb = ((size_t)16 * K * 2 + 255) / 256 * 256;
  const size_t s0 = ((size_t)16 * ng * 4 + 255) / 256 * 256;
  const size_t y3 = (size_t)kLowbitMaxSplit * 16 * N * 4;
  return xb + s0 + y3;
}

extern "C" int qs_lowbit_dequant(const uint8_t* packed, int64_t row_bytes, const void* scales,
                                 int scale_dtype, const void* zeros, int zero_dtype, float offset,
                                 int bits, int group_size, float* out, int64_t N, int64_t K,
                                 void* stream) {
  if (!packed || !scales || !out) return fail(QS_ERR_INVALID, "lowbit_dequant: null pointer");
  if (bits != 2 && bits != 3 && bits != 4) return fail(QS_ERR_UNSUPPORTED, "lowbit_dequant: bits 2, 3 or 4");
  if (group_size <= 0 || N <= 0 || K <= 0 || row_bytes < (K * bits + 7) / 8)
    return fail(QS_ERR_INVALID, "lowbit_dequant: bad shape");
  LowbitParams p{};
  p.packed = packed;
  p.row_bytes = row_bytes;
  p.scales = scales;
  p.zeros = zeros;
  p.scale_f16 = scale_dtype == QS_F16;
  p.zero_f16 = zero_dtype == QS_F16;
  p.offset = offset;
  p.N = (int)N;
  p.K = (int)K;
  p.ng = (int)((K + group_size - 1) / group_size);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (K % 4 == 0 && group_size % 4 == 0 && aligned(out, 16))
    hipLaunchKernelGGL(k_lowbit_dequant4<kLowbitDequantPieces>,
                       dim3((unsigned)cdiv(N * (K / 4), 256 * kLowbitDequantPieces)), dim3(256), 0, s, p, bits,
                       group_size, out);
  else
    hipLaunchKernelGGL(k_lowbit_dequant, dim3((unsigned)cdiv(N * K, 256)), dim3(256), 0, s, p, bits, group_size, out);
  return hip_check(hipGetLastError(), "k_lowbit_dequant launch");
}
