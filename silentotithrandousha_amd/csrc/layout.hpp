// Resident layout of MXFP4 matrices in HBM (host + device).
//
// Checkpoint layout (weights.rs:17-27): blocks [R][NB][16] u8, scales [R][NB] u8, with
// NB = cols/32 blocks of 32 E2M1 nibbles per row.
//
// Resident ("tile16") layout, chosen for the bf16 MFMA GEMV (v_mfma_f32_16x16x32_bf16):
// rows are grouped in tiles of 16. One wavefront owns one tile and walks it in NS =
// ceil(NB/4) steps; in step s lane l (0..63) needs block b = 4s + (l >> 4) of row
// 16t + (l & 15), so the lane's 16-byte load is exactly one MXFP4 block and the 64 lanes
// of a step read 1024 contiguous bytes:
//
//   weights: chunk (t, s, l) at byte  t*256*NB + (s*64 + l)*16          (valid iff b < NB)
//            Valid chunks of a tile are a contiguous prefix, so the weight region is the
//            checkpoint's size exactly: R*NB*16 bytes.
//   scales:  after the weight region, one 32-bit word per (t, q, l), q = 0..NQ-1 with
//            NQ = ceil(NS/4); byte i of the word is the E8M0 scale of step 4q+i for lane l
//            (0 where the step or block does not exist).  Word at  (t*NQ + q)*64 + l.
//
// The repack is a permutation of 16-byte blocks plus a permutation of scale bytes, so it is
// lossless; moe_dequant_expert_device decodes the resident copy back to the logical layout.
#pragma once
#include <stddef.h>
#include <stdint.h>

#if defined(__HIPCC__)
#define MOE_HD __host__ __device__ inline
#else
#define MOE_HD inline
#endif

namespace moe {

struct PackDims {
  uint32_t rows;   // R (multiple of 16)
  uint32_t nb;     // blocks per row (cols / 32)
  uint32_t ns;     // steps per tile = ceil(nb / 4)
  uint32_t nq;     // scale words per lane per tile = ceil(ns / 4)
  uint32_t tiles;  // R / 16
};

MOE_HD PackDims pack_dims(size_t rows, size_t cols) {
  PackDims d;
  d.rows = (uint32_t)rows;
  d.nb = (uint32_t)(cols / 32);
  d.ns = (d.nb + 3) / 4;
  d.nq = (d.ns + 3) / 4;
  d.tiles = (uint32_t)(rows / 16);
  return d;
}

MOE_HD size_t pack_weight_bytes(const PackDims &d) { return (size_t)d.rows * d.nb * 16; }
MOE_HD size_t pack_scale_bytes(const PackDims &d) { return (size_t)d.tiles * d.nq * 256; }
MOE_HD size_t pack_total_bytes(const PackDims &d) {
  return pack_weight_bytes(d) + pack_scale_bytes(d);
}

// Per-expert resident record: [gate_up packed][down packed][gate_up bias f32][down bias f32],
// every part 256-byte aligned; experts of a layer are `stride` bytes apart.
struct ExpertLayout {
  PackDims gu, dn;
  size_t gu_off, dn_off, gub_off, dnb_off, stride;
};

MOE_HD size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

MOE_HD ExpertLayout expert_layout(size_t hidden, size_t inter) {
  ExpertLayout L;
  L.gu = pack_dims(2 * inter, hidden);
  L.dn = pack_dims(hidden, inter);
  size_t off = 0;
  L.gu_off = off;
  off = align_up(off + pack_total_bytes(L.gu), 256);
  L.dn_off = off;
  off = align_up(off + pack_total_bytes(L.dn), 256);
  L.gub_off = off;
  off = align_up(off + 2 * inter * sizeof(float), 256);
  L.dnb_off = off;
  off = align_up(off + hidden * sizeof(float), 256);
  L.stride = align_up(off, 4096);
  return L;
}

}  // namespace moe
