// dm_layout.h -- HBM layouts of one uploaded MoE layer, shared by the host
// upload code and the kernels.
//
// The caller hands weights over in the reference's 4-bit layout
// (src/format/quant_reader.mojo:171-341): per tensor, fp16 group scales
// [N/G] and packed bytes [N/2], element i in byte i/2 (low nibble = even i),
// groups of G in {32, 64, 128, 256} consecutive elements along the flattened
// row-major index, codes signed int4 in [-7, 7].  At upload each matrix is
// re-tiled once into the "A16" layout below, with one scale per 32 columns
// (a source group's scale repeated over its 32-column chunks), so that one
// 16-byte load per lane feeds four MFMA k-steps and one 8-byte load carries
// the matching four fp16 scales.
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __HIPCC__
#define DM_HD __host__ __device__ __forceinline__
#else
#define DM_HD inline
#endif

namespace dm {

constexpr int kGroup = 32;        // G: elements per scale group (= MFMA k-step)
constexpr int kTileRows = 16;     // rows per A16 tile (MFMA M)
constexpr int kGroupsPerQuad = 4; // groups per 16-byte lane chunk
constexpr int kQuadCols = kGroup * kGroupsPerQuad;  // 128 columns per chunk

// ---- A16: 4-bit matrix W[R][C], R % 16 == 0, C % 128 == 0 ----------------
// Tile (rb, gq) covers rows 16*rb..16*rb+15 and groups 4*gq..4*gq+3.
// Lane l (0..63) of the tile owns row 16*rb + (l & 15) and, for each of the
// four groups c, the eight columns 32*(4*gq+c) + 8*(l >> 4) + kk, kk = 0..7:
// this is the A-operand layout of v_mfma_f32_16x16x32_bf16.
//   nibbles: 16 bytes per lane at a16_nib_offset(); word c holds group c.
//   Inside word c the nibble slot p (bits 4p..4p+3) holds kk = 2*(p&3) + (p>>2),
//   stored offset-binary u = q + 8, so (w >> 4i) & 0x000F000F yields the
//   column pair (2i, 2i+1) in the two 16-bit halves.
//   scales: fp16 [rb][gq][r][c], 8 bytes per row r at a16_sc_offset().
DM_HD size_t a16_nib_offset(int nGQ, int rb, int gq, int lane) {
  return ((size_t)(rb * nGQ + gq) * 64 + lane) * 16;
}
DM_HD size_t a16_sc_offset(int nGQ, int rb, int gq, int r) {
  return ((size_t)(rb * nGQ + gq) * 16 + r) * 4;
}
DM_HD int a16_slot_of_kk(int kk) { return (kk & 1) * 4 + (kk >> 1); }
DM_HD size_t a16_nib_bytes(int R, int C) { return (size_t)R * C / 2; }
DM_HD size_t a16_sc_count(int R, int C) { return (size_t)R * C / kGroup; }

// ---- R16: bf16 router matrix W[E'][H], H % 128 == 0 ----------------------
// Element (e, k) with k = 16*j + l sits at ((e*(H/128) + j/8)*16 + l)*8 + j%8,
// so the chain of lane l (k = l, l+16, l+32, ...) is 16-byte contiguous per
// eight steps and 16 lanes of one row read 256 consecutive bytes.
DM_HD size_t r16_index(int H, int e, int k) {
  int l = k & 15, j = k >> 4;
  return (((size_t)e * (H / 128) + (j >> 3)) * 16 + l) * 8 + (j & 7);
}

// ---- one uploaded layer ---------------------------------------------------
struct LayerDev {
  int H, E, K, I, Ish;
  const uint16_t* router;   // R16 bf16, E+1 rows: rows 0..E-1 router, row E shared-expert gate
  const uint8_t* gu_nib;    // per expert: A16 gate [I][H] then A16 up [I][H]
  const uint16_t* gu_sc;
  const uint8_t* d_nib;     // per expert: A16 down [H][I]
  const uint16_t* d_sc;
  const uint8_t* sgu_nib;   // shared expert: A16 gate [Ish][H] then up [Ish][H]
  const uint16_t* sgu_sc;
  const uint8_t* sd_nib;    // shared expert: A16 down [H][Ish]
  const uint16_t* sd_sc;
};

// ---- RMSNorm at the block edge ---------------------------------------------
// rmsnorm (src/layers/rmsnorm.mojo:10-48) of the block input:
// out = x / sqrt(sum(x * x) / H + eps) * gamma, each step rounded as written.
constexpr int kNormMaxH = 8192;  // largest H of the block-edge norm
struct NormSpec {
  float eps;           // > 0: the block sees the normalised input; 0: no norm
  const float* gamma;  // [H] fp32 post_attention_layernorm gamma (ones when unset)
  int seq;             // 1: the sum of squares in element order, as the reference
                       // sums it; 0: 256 strided partials and a halving tree
};

// ---- first-error keys ------------------------------------------------------
// Every check in the kernels that would raise in the reference records a
// 64-bit key with an integer atomicMin; the smallest key is the error the
// reference would have raised first.  A sync key (a bounded wait that gave
// up) sorts before all of them: the launch's outputs are then not valid and
// no other key of it can be trusted.  Its checks run: activation scan, router
// weight scan, logits (token, expert), softmax per token (max, exp per
// expert, sum), top-k per token, routed experts per (token, k) with rows j
// (gate, up, product) then outputs d, the shared expert per token, the shared
// gate per token, and the aggregation per (token, d).
//   [63:60] phase  [59:40] token  [39:32] slot  [31:4] pos  [3:0] kind
enum : uint32_t {
  kPhSync = 0,  // a wait between workgroups gave up: the outputs are not valid
  kPhX = 1, kPhRouterW = 2, kPhLogit = 3, kPhSoftmax = 4, kPhTopk = 5,
  kPhExpert = 6, kPhShared = 7, kPhGate = 8, kPhAgg = 9,
};
enum : uint32_t {  // kinds
  kTkSum = 0, kTkLeak = 1,                          // top-k
  kEkGate = 0, kEkUp = 1, kEkH = 2, kEkDown = 3,    // experts
  kEkBadId = 4,     // an expert id outside [0, E) given to the experts entry point
  kEkRecheck = 15,  // fused decode: a non-finite output whose first failing check is re-derived
  kGkLogit = 0, kGkRange = 1,                       // shared gate
};
constexpr uint64_t kNoError = ~0ull;

// Every wait of a persistent kernel on another workgroup's word is bounded:
// this many polls (each followed by s_sleep 1, about one second in all) by
// default, then a sync error is recorded and the wait ends.
constexpr long kDefaultSpinLimit = 1l << 20;

DM_HD uint64_t err_key(uint32_t phase, uint32_t token, uint32_t slot, uint32_t pos,
                       uint32_t kind) {
  return ((uint64_t)(phase & 0xF) << 60) | ((uint64_t)(token & 0xFFFFF) << 40) |
         ((uint64_t)(slot & 0xFF) << 32) | ((uint64_t)(pos & 0xFFFFFFF) << 4) |
         (uint64_t)(kind & 0xF);
}
DM_HD uint32_t key_phase(uint64_t k) { return (uint32_t)(k >> 60); }
DM_HD uint32_t key_token(uint64_t k) { return (uint32_t)(k >> 40) & 0xFFFFF; }
DM_HD uint32_t key_slot(uint64_t k) { return (uint32_t)(k >> 32) & 0xFF; }
DM_HD uint32_t key_pos(uint64_t k) { return (uint32_t)(k >> 4) & 0xFFFFFFF; }
DM_HD uint32_t key_kind(uint64_t k) { return (uint32_t)k & 0xF; }

}  // namespace dm
