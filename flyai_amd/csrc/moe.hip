// MXFP4 expert FFN for GPT-OSS: re-pack, gate_up (+ fused SwiGLU) and down kernels.
//
// Packed layout of one MXFP4 weight W[E][N][K] (N output rows, K inputs, G = K/32 blocks/row):
//   data   : [E][N/16 tiles][G*256 bytes].  Within a tile, group kg covers blocks 4kg..4kg+3 and
//            sits at byte kg*1024: lane l = 16*g + r holds the 16 bytes (32 E2M1 codes) of row r,
//            block 4kg+g.  A wave's 16-byte load per lane therefore reads one contiguous KiB.  The
//            last group holds only the G-4*(KG-1) existing blocks (no padding in the data).
//   scales : [E][N/16][KG4*256 bytes] after all data; dword (kg4, lane) holds the E8M0 scales of
//            (row r, block 4kg+g) for kg = 4kg4 .. 4kg4+3 in bytes 0..3 (0 past the end).
//
// The MFMA (v_mfma_f32_16x16x32_bf16) sees activations as A (16 rows x 32 K) and dequantised
// weights as B (32 K x 16 output features).  Because any consistent permutation of K is allowed
// in a dot product, lane (r, g) supplies, at MFMA step j of group kg, the 8 K values
// 32*(4kg+g) + 8j .. +7 for BOTH operands: the lane's 16 weight bytes feed four MFMA steps and
// its activation bytes are the matching 64 contiguous bytes of the activation row.
#include <atomic>
#include <type_traits>

#include "common.h"

namespace flyai {

struct MxGeom {
  int NT, G, KG, KG4;
  size_t data_bytes;  // whole data region (all experts)
};

__host__ __device__ inline MxGeom mx_geom(int E, int N, int K) {
  MxGeom g;
  g.NT = N / 16;
  g.G = K / 32;
  g.KG = (g.G + 3) / 4;
  g.KG4 = (g.KG + 3) / 4;
  g.data_bytes = (size_t)E * g.NT * g.G * 256;
  return g;
}

// ---- re-pack: HF blocks [E][N][G][16] + scales [E][N][G] -> tile layout -------------------------
__global__ __launch_bounds__(256) void mxfp4_repack_kernel(const uint8_t* __restrict__ blocks,
                                                           const uint8_t* __restrict__ scales,
                                                           int E, int N, int K,
                                                           uint8_t* __restrict__ packed) {
  const MxGeom gm = mx_geom(E, N, K);
  const size_t total = (size_t)E * gm.NT * gm.KG * 64;
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const int lane = idx % 64;
  const int kg = (idx / 64) % gm.KG;
  const size_t et = idx / 64 / gm.KG;  // e * NT + nt
  const int nt = et % gm.NT;
  const int e = et / gm.NT;
  const int r = lane & 15, g = lane >> 4;
  const int row = nt * 16 + r, blk = kg * 4 + g;
  if (blk < gm.G) {
    const uint4 v = *reinterpret_cast<const uint4*>(blocks + (((size_t)e * N + row) * gm.G + blk) * 16);
    *reinterpret_cast<uint4*>(packed + et * gm.G * 256 + (size_t)kg * 1024 + lane * 16) = v;
  }
  if ((kg & 3) == 0) {
    uint32_t word = 0;
    for (int i = 0; i < 4; ++i) {
      const int b2 = (kg + i) * 4 + g;
      if (kg + i < gm.KG && b2 < gm.G)
        word |= (uint32_t)scales[((size_t)e * N + row) * gm.G + b2] << (8 * i);
    }
    reinterpret_cast<uint32_t*>(packed + gm.data_bytes + et * gm.KG4 * 256)[(kg / 4) * 64 + lane] = word;
  }
}

// ---- expert kernels ---------------------------------------------------------------------------
// Workgroup = 4 waves = 4*NTW weight tiles (16 output rows each) of one expert, full K.  The
// expert's activation rows are staged in LDS, kRowsPerPass at a time, with fully coalesced loads
// (one pass serves every tile of the workgroup), so the only vector-memory loads in the K loop are
// the weights: 1 KiB per tile per group of 128 K, streamed through a DEPTH-deep register ring with
// non-temporal loads (DEPTH - 1 groups in flight while one computes).  Each group is dequantised in
// registers (gfx950 v_cvt_scalef32_pk_bf16_fp4, E8M0 scale in the exponent field) and fed to v_mfma_f32_16x16x32_bf16 with the activation
// fragment read from LDS (rows >= the pass's row count read as zero).  Larger groups take further
// passes over the weights.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// Buffer resource word 3 for raw (unformatted, unswizzled) loads on gfx9, and an offset past any
// resource this file builds (such a load returns zero and touches no memory).
constexpr int kBufRsrcWord3 = 0x00020000;
constexpr uint32_t kBufOutside = 0x80000000u;

// 16 bytes through a buffer resource, nontemporal
__device__ __forceinline__ uint4 buf_ld16_nt(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 2);
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint4 ld_nt(const uint8_t* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float swiglu_gptoss(float gate, float up) {
  // modeling_gpt_oss.py:82-88: gate clamped above at 7, up clamped to [-7, 7]
  const float g = fminf(gate, 7.0f);
  const float u = fminf(fmaxf(up, -7.0f), 7.0f);
  const float glu = g * __builtin_amdgcn_rcpf(1.0f + __expf(-1.702f * g));
  return (u + 1.0f) * glu;
}

// value of lane ^ 1 (DPP quad permutation [1, 0, 3, 2]; no LDS traffic)
__device__ __forceinline__ float lane_xor1(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
}

// The gate_up epilogue for one 16-feature tile's 4 rows held by lane (r, g) (rows 4g + v, v < 4):
// lanes r and r ^ 1 hold the gate (even r) and up values of one output feature.  One exchange of two
// values each gives the even lane (gate, up) of rows v = 0, 1 and the odd lane those of rows v = 2, 3,
// so every lane computes two SwiGLUs (none twice) and stores two results: store(v, bf16 bits).
template <class Store>
__device__ __forceinline__ void swiglu_pairs(const float (&val)[4], int r, const Store& store) {
  const bool ev = (r & 1) == 0;
  const float s0 = lane_xor1(ev ? val[2] : val[0]);
  const float s1 = lane_xor1(ev ? val[3] : val[1]);
  store(ev ? 0 : 2, f2bf(swiglu_gptoss(ev ? val[0] : s0, ev ? s0 : val[2])));
  store(ev ? 1 : 3, f2bf(swiglu_gptoss(ev ? val[1] : s1, ev ? s1 : val[3])));
}

// compile-time loop: f(integral_constant<int, B>) ... f(integral_constant<int, N-1>)
template <int B, int N, class F>
__device__ __forceinline__ void mx_static_for(F&& f) {
  if constexpr (B < N) {
    f(std::integral_constant<int, B>{});
    mx_static_for<B + 1, N>(f);
  }
}

constexpr int kRowsPerPass = 8;

__host__ __device__ inline int mx_lds_row_bytes(int K) { return K * 2 + 16; }  // +16 B vs bank conflicts

template <bool GATE_UP, int NTW, int DEPTH>
__global__ __launch_bounds__(256, 3) void moe_mxfp4_kernel(
    const uint16_t* __restrict__ act, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ offsets, int k_top, const uint8_t* __restrict__ packed,
    const float* __restrict__ bias, int E, int N, int K, int min_rows, int max_rows,
    void* __restrict__ out) {
  extern __shared__ uint4 xs_lds[];  // [kRowsPerPass][K*2+16 bytes]
  const MxGeom gm = mx_geom(E, N, K);
  constexpr int kTilesPerWG = 4 * NTW;
  const int wg_per_e = (gm.NT + kTilesPerWG - 1) / kTilesPerWG;
  const int e = blockIdx.x / wg_per_e;
  const int wgi = blockIdx.x % wg_per_e;
  const int row_lo = offsets[e];
  const int n_e = offsets[e + 1] - row_lo;
  if (n_e <= 0 || n_e < min_rows || n_e > max_rows) return;  // uniform over the workgroup
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nt0 = wgi * kTilesPerWG + wave * NTW;
  const int ntw = max(0, min(NTW, gm.NT - nt0));  // waves past the last tile still join the barriers
  const int r = lane & 15, g = lane >> 4;
  const int row_bytes = mx_lds_row_bytes(K);
  const int row_vecs = K / 8;  // 16-byte vectors per activation row
  const bool k_pow2 = (k_top & (k_top - 1)) == 0;  // slot -> token by a shift (the routers' k: 2, 4, 8)
  const int k_shift = __builtin_ctz((unsigned)k_top);

  // The wave's weight tiles and scale dwords through buffer resources: a load outside the valid
  // range (the last ring body's groups past KG, a block past the row's end, a tile past the
  // expert's last) gets an offset past the resource and reads zero with no memory access.  The
  // loads are therefore unconditional: no branch separates a load from the ring, so the compiler's
  // waits count the ring exactly (with the loads under branches it drained the ring at every body).
  const int tile_stride = gm.G * 256;
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(packed + ((size_t)e * gm.NT + nt0) * tile_stride), (short)0, ntw * tile_stride,
      kBufRsrcWord3);
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(packed + gm.data_bytes + ((size_t)e * gm.NT + nt0) * gm.KG4 * 256), (short)0,
      ntw * gm.KG4 * 256, kBufRsrcWord3);
  const char* lds = reinterpret_cast<const char*>(xs_lds);

  auto load_w = [&](uint4 (&w)[NTW], int kg) {
    const bool bvalid = kg < gm.KG && 4 * kg + g < gm.G;
#pragma unroll
    for (int n = 0; n < NTW; ++n)
      w[n] = buf_ld16_nt(wrs, bvalid ? (uint32_t)(n * tile_stride + kg * 1024 + lane * 16) : kBufOutside);
  };
  auto load_sc = [&](uint32_t (&sc)[NTW], int kg4) {
#pragma unroll
    for (int n = 0; n < NTW; ++n)
      sc[n] = __builtin_amdgcn_raw_buffer_load_b32(
          srs, kg4 < gm.KG4 ? (uint32_t)(n * gm.KG4 * 256 + kg4 * 256 + lane * 4) : kBufOutside, 0, 0);
  };
  // Static bodies of DEPTH groups: a DEPTH-deep weight ring (DEPTH - 1 groups in flight while one
  // computes) and the next body's scale dwords loaded one body ahead, so no wait drains the ring.
  static_assert(DEPTH % 4 == 0, "a body covers whole scale dwords (4 groups each)");
  constexpr int kSc = DEPTH / 4;
  uint4 w[DEPTH][NTW];
  uint32_t sc_cur[kSc][NTW], sc_nxt[kSc][NTW];
  // The tiles' bias, loaded with the first pass's staging: requested ahead of the weight ring, so the
  // epilogue does not pay a global round trip of its own.
  float bias_r[NTW];

  for (int m0 = 0; m0 < n_e; m0 += kRowsPerPass) {
    const int rows = min(kRowsPerPass, n_e - m0);
    lds_barrier();  // the previous pass is done with the LDS rows
    // staging loads go out in batches of kStageBatch per thread (one round trip per batch, not per
    // vector); indices past the end are clamped for the load and not stored.  Batches of 5
    // measured 4% slower than 4 on the 9-layer decode step (32 sequences, 56 tokens).  The pass's
    // first weight groups are requested right after the first batch, so the weight stream does not
    // wait for the activation round trip; the LDS-only barrier below leaves them in flight.
    constexpr int kStageBatch = 4;
    const int total = rows * row_vecs;
    // (row, vector) of the thread's element b0 + j * 256 + tid, stepped by 256 without an integer
    // division (a 32-bit division is ~25 VALU instructions, and these sit before the first load)
    int cr = 0, cv = threadIdx.x;
    while (cv >= row_vecs) {
      cv -= row_vecs;
      ++cr;
    }
    for (int b0 = 0; b0 < total; b0 += kStageBatch * 256) {
      u32x4_t v4[kStageBatch];
      int jr[kStageBatch], jv[kStageBatch];
#pragma unroll
      for (int j = 0; j < kStageBatch; ++j) {
        jr[j] = cr;
        jv[j] = cv;
        const bool in = cr < rows;  // element index < total; past it, the last element (not stored)
        const int rr = in ? cr : rows - 1, v = in ? cv : row_vecs - 1;
        const int p = row_lo + m0 + rr;
        const int src = GATE_UP ? (k_pow2 ? perm[p] >> k_shift : perm[p] / k_top) : p;
        v4[j] = reinterpret_cast<const u32x4_t*>(act + (size_t)src * K)[v];
        cv += 256;
        while (cv >= row_vecs) {
          cv -= row_vecs;
          ++cr;
        }
      }
      if (m0 == 0 && b0 == 0) {
#pragma unroll
        for (int n = 0; n < NTW; ++n) bias_r[n] = n < ntw ? bias[(size_t)e * N + (nt0 + n) * 16 + r] : 0.f;
      }
      if (b0 == 0) {
        mx_static_for<0, kSc>([&](auto q) { load_sc(sc_cur[q], q); });
        mx_static_for<0, DEPTH - 1>([&](auto j) { load_w(w[j], j); });
      }
#pragma unroll
      for (int j = 0; j < kStageBatch; ++j)
        if (jr[j] < rows)
          *reinterpret_cast<u32x4_t*>(const_cast<char*>(lds) + jr[j] * row_bytes + jv[j] * 16) = v4[j];
    }
    lds_barrier();
    if (ntw == 0) continue;
    const bool aval = r < rows;
    const char* arow = lds + r * row_bytes + 64 * g;

    f32x4_t acc[NTW];
#pragma unroll
    for (int n = 0; n < NTW; ++n) acc[n] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // byte b of sc[n] is the E8M0 scale of group 4*kg4 + b
    auto compute = [&](const uint4 (&wg)[NTW], const uint32_t (&sc)[NTW], int kg, int b) {
      uint4 a[4];
      const bool ok = aval && kg < gm.KG && 4 * kg + g < gm.G;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        a[j] = ok ? *reinterpret_cast<const uint4*>(arow + 256 * kg + 16 * j) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int n = 0; n < NTW; ++n) {
        const float scale = e8m0_operand((sc[n] >> (8 * b)) & 0xffu);
        const uint32_t wd[4] = {wg[n].x, wg[n].y, wg[n].z, wg[n].w};
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[n] = mfma16x16x32(as_bf16x8(a[j]), fp4x8_to_bf16x8(wd[j], scale), acc[n]);
      }
    };

    for (int kg0 = 0; kg0 < gm.KG; kg0 += DEPTH) {
      mx_static_for<0, kSc>([&](auto q) { load_sc(sc_nxt[q], kg0 / 4 + kSc + q); });
      mx_static_for<0, DEPTH>([&](auto j) {
        load_w(w[(j + DEPTH - 1) % DEPTH], kg0 + j + DEPTH - 1);
        compute(w[j], sc_cur[j / 4], kg0 + j, j % 4);
      });
      mx_static_for<0, kSc>([&](auto q) {
#pragma unroll
        for (int n = 0; n < NTW; ++n) sc_cur[q][n] = sc_nxt[q][n];
      });
    }

    // epilogue: lane holds D[act row 4g+v][feature r] of each tile
#pragma unroll
    for (int n = 0; n < NTW; ++n) {
      const int feat = (nt0 + n) * 16 + r;
      const bool nval = n < ntw;
      const float bsum = bias_r[n];
      if (GATE_UP) {
        const float val[4] = {acc[n][0] + bsum, acc[n][1] + bsum, acc[n][2] + bsum, acc[n][3] + bsum};
        swiglu_pairs(val, r, [&](int v, uint16_t hbits) {
          if (nval && 4 * g + v < rows)
            reinterpret_cast<uint16_t*>(out)[(size_t)(row_lo + m0 + 4 * g + v) * (N / 2) + feat / 2] = hbits;
        });
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int orow = 4 * g + v;
          if (nval && orow < rows)
            reinterpret_cast<float*>(out)[(size_t)(row_lo + m0 + orow) * N + feat] = acc[n][v] + bsum;
        }
      }
    }
  }
}

// Weight tiles per wave and weight-ring depth (128-K groups) of the decode-sized kernels.  Two tiles
// and an 8-deep ring keep 14 KiB in flight per wave at 3 waves per SIMD (166 registers), against
// 9 KiB for 3 tiles and a 4-deep ring (162 registers); the workgroups are also a third smaller, so
// the end of the launch, where the last workgroups run alone, is shorter.  Measured on the 9-layer
// decode step of 32 sequences, 56 tokens (A/B on one box): 3 tiles x 4 deep 3.13 ms; 2 x 8 3.04 ms; 1 x 8, 2 x 4 and 2 x 12 for
// gate_up and 1 x 8, 1 x 16 and 2 x 12 for down all slower.
constexpr int kNTWGateUp = 2;
constexpr int kNTWDown = 2;
constexpr int kDepthGateUp = 8;
constexpr int kDepthDown = 8;

// ---- dense groups as a tiled GEMM ----------------------------------------------------------------
// For groups of many rows the weights are still read once from HBM, but each weight byte now feeds
// up to 96 rows, so the kernel must keep HBM busy and the MFMA pipes busy at the same time.
// A workgroup of 8 waves (2 per SIMD, the CU's whole LDS) computes, for one expert and 96 of its
// rows, a chunk of consecutive 256-row weight blocks (16 packed tiles each); wave w owns tiles
// 2w, 2w+1 of the block and all 6 row tiles (12 accumulators; every A fragment feeds 2 MFMAs,
// every B fragment 6).  The blocks of a chunk share the activation rows, so the load pipeline runs
// on across block boundaries and a workgroup's start-up latency (index loads, pipeline fill) is
// paid once per chunk, not once per block.  K advances one 128-K group at a time:
//  * the weights (1 KiB per tile and group) go global -> registers through a 4-deep ring, each wave
//    loading only its own tiles, as the memory-bound kernels do: registers hold far more bytes in
//    flight than LDS could;
//  * the activation rows (shared by all 8 waves) and the weight scales go global -> LDS directly
//    (global_load_lds) through 4 stages of 28 KiB; a group's loads are issued 3 groups ahead;
//  * activations sit in LDS row-major, a row tile (16 rows x 128 K) in 4 KiB, each row's sixteen
//    16-byte chunks XOR-swizzled by the row: chunk c of row r at position c ^ act_swz(r).  Each
//    direct-to-LDS load fills 4 whole rows (16 consecutive lanes read one row's 256 contiguous
//    bytes); a fragment-order load (16 rows x 16 B per lane group) streams from L2 at a third of
//    the rate.  Lane (g, r) = (lane / 16, lane % 16) feeds step j of row tile m with row 16m + r,
//    K = 32g + 8j of the group, read from position (4g + j) ^ act_swz(r), which is conflict-free
//    under the rule act_swz states;
//  * the stages are separate LDS arrays with compile-time stage numbers, so the compiler can tell
//    a stage's reads from the asynchronous writes into the other stages; each stage is waited for
//    with an explicit vmcnt that leaves the 2 younger groups' loads in flight (vector-memory loads
//    complete in issue order, so within a group the register loads go out before the LDS ones),
//    and the barrier is a bare s_barrier after the wave's own LDS reads (__syncthreads() would
//    also wait for every outstanding global load);
//  * a group is 4 MFMA steps of 32 K; the LDS reads and fp4 conversions of step j+1 are issued
//    under the 12 MFMAs of step j (operands are double-buffered in registers, never copied), and
//    the barrier that hands over the next stage sits before the last step, so the next group's
//    first reads hide under that step's MFMAs;
//  * packed MXFP4 is dequantised per wave (v_cvt_scalef32_pk_bf16_fp4) right before its MFMAs.
// Each block runs its K groups padded to a multiple of 4, so blocks start on stage 0 and the
// 4-way unrolled group loop is straight-line; a block's outputs are written after its last group.
// Loads are unconditional with clamped addresses: rows past the group read row 0 and are never
// stored; weight lanes past a row's last block (and the padding groups) are zeroed before
// conversion, their activation slots read the row's first group (finite values); tiles past N
// load a clamped tile whose codes are zeroed before conversion (MFMAs on zero operands draw less
// power: down at 128 experts x 65 rows 194-195 -> 192 us) and are never stored; the 3 groups issued
// past the chunk's end read clamped addresses and are never computed on.
constexpr int kGemmTiles = 16;                       // packed 16-row weight tiles per block
constexpr int kGemmRows = 96;                        // group rows per pass
constexpr int kGemmStage = kGemmRows * 256 + kGemmTiles * 256;  // activations + scale dwords
constexpr int kGemmStages = 4;

// instruction classes for __builtin_amdgcn_sched_group_barrier
constexpr int kSchedValu = 0x2, kSchedMfma = 0x8, kSchedVmem = 0x10, kSchedDsRead = 0x100;

// Position key of activation row r (0..15) in the dense GEMM's LDS row tiles: the chunk c of row r sits
// at 16-byte slot c ^ act_swz(r).  gfx950's LDS has 64 banks of 4 bytes, and a ds_read_b128 serves
// the 64 lanes in four cycles of 16, each a half-wave's lane quads of one parity (quads 0, 3, 5, 6 of
// the half together, then quads 1, 2, 4, 7); it is conflict-free when the 16 lanes of each cycle read
// 16 different slots of a 256-byte row (measured with single-lane pairs and the conflict counter).
// Lane (g, r) reads slot (4g + j) ^ act_swz(r).  A cycle holds lanes of g = 2h with r in one class
// of (r2 ^ r3) and lanes of g = 2h + 1 with r in the other (r2, r3 the bits of r), and their chunks
// differ in bit 2.  act_swz maps each class onto a set closed under ^4 ({0..7} and {8..15}), so
// the two halves of a cycle land on complementary slot sets.  (Keying by r itself put lanes 0-3
// and 20-23 on the same slots: a 2-way conflict on every read.)
__device__ __forceinline__ int act_swz(int r) {
  return (r & 3) | ((r >> 1) & 4) | ((((r >> 2) ^ (r >> 3)) & 1) << 3);
}

// Work units of the dense GEMMs: every group of at least min_rows rows is cut into passes of
// kGemmRows rows, the passes are numbered expert by expert, and unit u is weight-block chunk
// u % chunks_per_e of pass u / chunks_per_e.  A group of many rows (a hot expert) so spreads its
// passes over workgroups instead of running them one after another in each of its workgroups.  Every
// workgroup derives the numbering from offsets[0..E] (an exclusive scan in LDS); the grid is sized for
// the most passes any routing can give, sum_e ceil(n_e / kGemmRows) <= rows_total / kGemmRows + E, and
// units past the last pass exit.

struct DenseUnit {
  int e, m0, rows, row_lo, n_e;
};

// The unit of this workgroup; false: none (uniform over the workgroup).  pre: E + 1 ints of LDS.  The
// live units are spread over the 8 XCDs, consecutive ones on one XCD (workgroups are dealt to the XCDs
// round-robin by index), so that an XCD's L2 serves a pass's activation rows to all its chunks and
// the units past the live count, which exit, do not leave XCDs idle.
__device__ __forceinline__ bool dense_unit(const int32_t* __restrict__ offsets, int E, int min_rows,
                                           int chunks_per_e, int* pre, DenseUnit& u, int& unit) {
  const int tid = threadIdx.x;
  if (tid < 64) {  // one wave: 4 experts per lane, scanned in order (E <= 256)
    int v[4], sum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = 4 * tid + j;
      const int n = e < E ? offsets[e + 1] - offsets[e] : 0;
      v[j] = (n > 0 && n >= min_rows) ? (n + kGemmRows - 1) / kGemmRows : 0;
      sum += v[j];
    }
    int incl = sum;
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(incl, o, 64);
      if (tid >= o) incl += y;
    }
    int run = incl - sum;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = 4 * tid + j;
      if (e < E) pre[e] = run;
      run += v[j];
    }
    if (tid == 63) pre[E] = incl;  // every pass (experts past E add none)
  }
  __syncthreads();  // no global load is in flight yet
  const int live = pre[E] * chunks_per_e;
  const int per_xcd = (live + 7) / 8;
  const int slot = (int)(blockIdx.x / 8);
  unit = (int)(blockIdx.x % 8) * per_xcd + slot;
  if (slot >= per_xcd || unit >= live) return false;
  const int p = unit / chunks_per_e;
  // the expert whose pass range holds p: the largest e with pre[e] <= p (pre is non-decreasing; an
  // expert with no passes shares its pre with the next, so the largest such e has passes); a fixed
  // 8-step search covers E <= 256 without a loop
  int e = 0;
#pragma unroll
  for (int step = 128; step > 0; step >>= 1)
    if (e + step < E && pre[e + step] <= p) e += step;
  u.e = e;
  u.row_lo = offsets[e];
  u.n_e = offsets[e + 1] - u.row_lo;
  u.m0 = (p - pre[e]) * kGemmRows;
  u.rows = min(kGemmRows, u.n_e - u.m0);
  return true;
}

// what one workgroup of the tiled GEMM works on: an expert, its rows, a chunk of weight blocks
struct GemmCtx {
  const uint16_t* act;
  const int32_t* perm;
  const float* bias;
  void* out;
  const uint8_t* wbase;  // the expert's packed tiles, + lane * 16
  const uint8_t* sbase;  // the expert's scale rows, + lane * 4
  MxGeom gm;
  size_t tile_bytes;
  int k_top, N, K, e, nb0, nbn, row_lo, lane, wave, r, g;
};

// The chunk's bias (nbn blocks of 256 features from block nb0) goes to LDS once per pass, every
// load before the first store.  The epilogues read it there: a register copy per block would need a
// global load in the loop, and waiting for it (vector-memory counts complete in issue order) would
// drain the groups prefetched behind it.
constexpr int kGemmBiasBlocks = 32;
__device__ __forceinline__ void stage_chunk_bias(const float* __restrict__ bias, int e, int N, int nb0, int nbn,
                                                 float (&bias_s)[kGemmBiasBlocks * 256]) {
  constexpr int kPer = kGemmBiasBlocks * 256 / 512;
  float v[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int i = (int)threadIdx.x + j * 512;
    const int f = nb0 * 256 + i;
    v[j] = (i < nbn * 256 && f < N) ? bias[(size_t)e * N + f] : 0.f;
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j) bias_s[threadIdx.x + j * 512] = v[j];
}

// One pass over MT row tiles (16*MT rows from m0) and every block of the chunk.
template <bool GATE_UP, int MT>
__device__ __forceinline__ void gemm_pass(const GemmCtx& c, char (&st0)[kGemmStage], char (&st1)[kGemmStage],
                                          char (&st2)[kGemmStage], char (&st3)[kGemmStage],
                                          float (&bias_s)[kGemmBiasBlocks * 256], int m0, int rows) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) void* lds_ptr;
  static_assert(MT >= 1 && MT <= 6, "row tiles per pass");
  constexpr int MD = (MT + 1) / 2;                    // activation DMA instructions (2 row tiles each)
  constexpr int ABYTES = MD * 8192;                   // activation part of a stage
  constexpr int LOADS = 2 + 2 + MD;                   // weight tiles, scale rows, activation blocks
  constexpr int WAIT = (kGemmStages - 2) * LOADS;     // loads younger than the stage waited for
  const MxGeom& gm = c.gm;
  const int lane = c.lane, wave = c.wave, r = c.r, g = c.g;
  const int sfrag_off = ABYTES + 2 * wave * 256 + lane * 4;
  // this wave's tile n of chunk block nb (clamped into the expert)
  auto tile_of = [&](int nb, int n) __attribute__((always_inline)) {
    return min((c.nb0 + nb) * kGemmTiles + 2 * wave + n, gm.NT - 1);
  };
  const int KGP = (gm.KG + kGemmStages - 1) / kGemmStages * kGemmStages;  // groups per block, padded

  // activation DMA: instruction J fills block b = J*8 + wave, rows 4 (b % 4) .. +3 of row tile b / 4:
  // lane L writes position L % 16 of row rt = 4 (b % 4) + L / 16 and so fetches 16-byte chunk
  // (L % 16) ^ act_swz(rt) of that row's 256 bytes (16 consecutive lanes read one row; an odd MT loads one
  // more row tile, of clamped rows, that no MFMA reads)
  const uint16_t* arow[MD];
  int ablk[MD];  // the 32-K block of the group the lane's chunk lies in
#pragma unroll
  for (int J = 0; J < MD; ++J) {
    const int b = J * 8 + wave;
    const int rt = 4 * (b & 3) + (lane >> 4);
    const int row = (b >> 2) * 16 + rt;
    const int p = c.row_lo + m0 + (row < rows ? row : 0);
    const int chunk = (lane & 15) ^ act_swz(rt);
    arow[J] = c.act + (size_t)(GATE_UP ? c.perm[p] / c.k_top : p) * c.K + chunk * 8;
    ablk[J] = chunk >> 2;
  }
  // step j's fragment of lane (g, r): row r, K 32g + 8j = chunk 4g + j at position (4g + j) ^ act_swz(r)
  const int afrag = r * 256 + (((4 * g) ^ act_swz(r)) << 4);
  // the next group to load: block i_nb of the chunk (past the end: the last block), group i_kg
  int i_nb = 0, i_kg = 0;
  // the loads of that group: weights into the ring slot, then scales and activations into the
  // stage; advances the position
  auto issue = [&](u32x4 (&bq)[2], char* stage) __attribute__((always_inline)) {
    const int nb = min(i_nb, c.nbn - 1), kg = i_kg;
    const bool blk = 4 * kg + g < gm.G;  // the lane's block of the group exists
    const size_t woff = blk ? (size_t)kg * 1024 : 0;
#pragma unroll
    for (int n = 0; n < 2; ++n)
      bq[n] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(c.wbase + (size_t)tile_of(nb, n) * c.tile_bytes + woff));
#pragma unroll
    for (int n = 0; n < 2; ++n)
      __builtin_amdgcn_global_load_lds((const void*)(c.sbase + ((size_t)tile_of(nb, n) * gm.KG4 + min(kg / 4, gm.KG4 - 1)) * 256),
                                       (lds_ptr)(stage + ABYTES + (2 * wave + n) * 256), 4, 0, 0);
    // a chunk past the row's last block (or of a padding group) reads the row's first group instead:
    // in bounds and finite, and multiplied only by zeroed weights
#pragma unroll
    for (int J = 0; J < MD; ++J) {
      const int col = 4 * kg + ablk[J] < gm.G ? kg * 128 : 0;
      __builtin_amdgcn_global_load_lds((const void*)(arow[J] + col), (lds_ptr)(stage + (J * 8 + wave) * 1024), 16, 0, 0);
    }
    if (++i_kg == KGP) {
      i_kg = 0;
      ++i_nb;
    }
  };
  f32x4_t acc[MT][2];
  auto zero_acc = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int n = 0; n < 2; ++n) acc[m][n] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  };
  zero_acc();

  // double-buffered step operands (x0 / x1), the weight ring, the current group's scales
  bf16x8_t a0[MT], a1[MT], b0[2], b1[2];
  u32x4 w0[2], w1[2], w2[2], w3[2];
  float scale[2];
  bool bok[2] = {false, false};
  int live_n = 2;  // this wave's tiles of the current block that lie inside the expert
  auto read_scales = [&](const char* stage, int kg) __attribute__((always_inline)) {
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      const uint32_t sw = *reinterpret_cast<const uint32_t*>(stage + sfrag_off + n * 256);
      scale[n] = e8m0_operand((sw >> (8 * (kg & 3))) & 0xffu);
    }
    // the lane's weight block exists and its tile lies inside the expert
#pragma unroll
    for (int n = 0; n < 2; ++n) bok[n] = 4 * kg + g < gm.G && n < live_n;
  };
  auto read_a = [&](bf16x8_t (&a)[MT], const char* stage, auto j) __attribute__((always_inline)) {
    const int fo = afrag ^ (int(j) << 4);
#pragma unroll
    for (int m = 0; m < MT; ++m) a[m] = as_bf16x8(*reinterpret_cast<const uint4*>(stage + m * 4096 + fo));
  };
  auto cvt = [&](bf16x8_t (&b)[2], const u32x4 (&bq)[2], auto j) __attribute__((always_inline)) {
#pragma unroll
    for (int n = 0; n < 2; ++n) b[n] = fp4x8_to_bf16x8(bok[n] ? bq[n][int(j)] : 0u, scale[n]);
  };
  auto mfma_step = [&](const bf16x8_t (&a)[MT], const bf16x8_t (&b)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int n = 0; n < 2; ++n) acc[m][n] = mfma16x16x32(a[m], b[n], acc[m][n]);
  };
  // 2*MT MFMAs with the next step's MT reads going out early and its 8 conversions spread after
  auto sched_step = [&]() __attribute__((always_inline)) {
    mx_static_for<0, MT>([&](auto) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    });
    mx_static_for<0, MT>([&](auto) {
      __builtin_amdgcn_sched_group_barrier(kSchedValu, 2, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
    });
    __builtin_amdgcn_sched_barrier(0);
  };
  // bias of this wave's two columns of chunk block nb
  float bsum[2];
  auto load_bias = [&](int nb) __attribute__((always_inline)) {
#pragma unroll
    for (int n = 0; n < 2; ++n) bsum[n] = bias_s[(tile_of(min(nb, c.nbn - 1), n) - c.nb0 * kGemmTiles) * 16 + r];
  };
  // acc[m][n][v] = D[group row 16m + 4g + v][feature (block tile 2*wave + n) * 16 + r]
  auto epilogue = [&](int nb) __attribute__((always_inline)) {
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      const int tile = (c.nb0 + nb) * kGemmTiles + 2 * wave + n;
      const bool nval = tile < gm.NT;
      const int feat = tile * 16 + r;
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        if (GATE_UP) {
          const float val[4] = {acc[m][n][0] + bsum[n], acc[m][n][1] + bsum[n], acc[m][n][2] + bsum[n],
                                acc[m][n][3] + bsum[n]};
          swiglu_pairs(val, r, [&](int v, uint16_t hbits) {
            const int orow = 16 * m + 4 * g + v;
            if (nval && orow < rows)
              reinterpret_cast<uint16_t*>(c.out)[(size_t)(c.row_lo + m0 + orow) * (c.N / 2) + feat / 2] = hbits;
          });
        } else {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int orow = 16 * m + 4 * g + v;
            if (nval && orow < rows)
              reinterpret_cast<float*>(c.out)[(size_t)(c.row_lo + m0 + orow) * c.N + feat] = acc[m][n][v] + bsum[n];
          }
        }
      }
    }
  };

  // group kg of a block from stage `cur` and weight slot `wc` (steps 0, 1, 2 from x0, x1, x0;
  // step 3 from x1); hands over to the next group (`nxt`, `wn`, into x0) and refills `cur` and
  // `wc` 4 groups ahead
  auto group = [&](char* cur, u32x4 (&wc)[2], const char* nxt, const u32x4 (&wn)[2], int kg)
                   __attribute__((always_inline)) {
    read_a(a1, cur, std::integral_constant<int, 1>{});
    cvt(b1, wc, std::integral_constant<int, 1>{});
    mfma_step(a0, b0);
    sched_step();
    read_a(a0, cur, std::integral_constant<int, 2>{});
    cvt(b0, wc, std::integral_constant<int, 2>{});
    mfma_step(a1, b1);
    sched_step();
    read_a(a1, cur, std::integral_constant<int, 3>{});
    cvt(b1, wc, std::integral_constant<int, 3>{});
    mfma_step(a0, b0);
    sched_step();
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(WAIT));  // this wave's loads of the next group are done
    lds_barrier();  // every wave's part of the next stage is in LDS; every wave is done with `cur`
    // step 3 under the next group's first reads and conversions and the refill
    read_scales(nxt, kg + 1 == KGP ? 0 : kg + 1);
    read_a(a0, nxt, std::integral_constant<int, 0>{});
    mfma_step(a1, b1);
    cvt(b0, wn, std::integral_constant<int, 0>{});
    issue(wc, cur);
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
    mx_static_for<0, MT>([&](auto) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    });
    mx_static_for<0, MT - 1>([&](auto) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedValu, 4, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedVmem, 2, 0);
    });
    __builtin_amdgcn_sched_barrier(0);
  };

  lds_barrier();  // every wave is done with the previous pass's stages (and the bias)
  stage_chunk_bias(c.bias, c.e, c.N, c.nb0, c.nbn, bias_s);
  // the stage waits count loads per group in issue order: no load may move across a group
  asm volatile("" ::: "memory");
  issue(w0, st0);
  asm volatile("" ::: "memory");
  issue(w1, st1);
  asm volatile("" ::: "memory");
  issue(w2, st2);
  asm volatile("" ::: "memory");
  issue(w3, st3);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(waitcnt_vm((kGemmStages - 1) * LOADS));
  lds_barrier();  // stage 0 is in LDS
  for (int nb = 0; nb < c.nbn; ++nb) {
    // the block's first operands (stage 0 stays valid until the first group's barrier); taken here
    // rather than carried through the previous block's epilogue, to keep that epilogue's register
    // pressure low: a spill would add vector-memory operations the stage waits do not count
    live_n = max(0, min(2, gm.NT - ((c.nb0 + nb) * kGemmTiles + 2 * wave)));
    read_scales(st0, 0);
    read_a(a0, st0, std::integral_constant<int, 0>{});
    cvt(b0, w0, std::integral_constant<int, 0>{});
    for (int kg = 0; kg < KGP; kg += kGemmStages) {
      group(st0, w0, st1, w1, kg);
      group(st1, w1, st2, w2, kg + 1);
      group(st2, w2, st3, w3, kg + 2);
      group(st3, w3, st0, w0, kg + 3);
    }
    load_bias(nb);
    epilogue(nb);
    zero_acc();
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // the loads past the chunk's end have landed
}

template <bool GATE_UP>
__global__ __launch_bounds__(512) void moe_mxfp4_gemm_kernel(
    const uint16_t* __restrict__ act, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ offsets, int k_top, const uint8_t* __restrict__ packed,
    const float* __restrict__ bias, int E, int N, int K, int min_rows, int chunk, void* __restrict__ out) {
  __shared__ __align__(16) char st0[kGemmStage];
  __shared__ __align__(16) char st1[kGemmStage];
  __shared__ __align__(16) char st2[kGemmStage];
  __shared__ __align__(16) char st3[kGemmStage];
  GemmCtx c;
  c.gm = mx_geom(E, N, K);
  const int blocks_per_e = (c.gm.NT + kGemmTiles - 1) / kGemmTiles;
  const int chunks_per_e = (blocks_per_e + chunk - 1) / chunk;
  __shared__ int pass_pre[257];
  __shared__ float bias_s[kGemmBiasBlocks * 256];
  DenseUnit du;
  int unit = 0;
  if (!dense_unit(offsets, E, min_rows, chunks_per_e, pass_pre, du, unit)) return;
  c.e = du.e;
  c.nb0 = (unit % chunks_per_e) * chunk;
  c.nbn = min(chunk, blocks_per_e - c.nb0);  // weight blocks in this chunk
  c.row_lo = du.row_lo;
  c.act = act;
  c.perm = perm;
  c.bias = bias;
  c.out = out;
  c.k_top = k_top;
  c.N = N;
  c.K = K;
  const int tid = threadIdx.x;
  c.lane = tid & 63;
  c.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  c.r = c.lane & 15;
  c.g = c.lane >> 4;
  c.tile_bytes = (size_t)c.gm.G * 256;
  c.wbase = packed + (size_t)c.e * c.gm.NT * c.tile_bytes + c.lane * 16;
  c.sbase = packed + c.gm.data_bytes + (size_t)c.e * c.gm.NT * c.gm.KG4 * 256 + c.lane * 4;
  // this unit's pass of up to 96 rows, as the fewest 16-row tiles that hold them (at least 2)
  if (du.rows > 80) gemm_pass<GATE_UP, 6>(c, st0, st1, st2, st3, bias_s, du.m0, du.rows);
  else if (du.rows > 64) gemm_pass<GATE_UP, 5>(c, st0, st1, st2, st3, bias_s, du.m0, du.rows);
  else if (du.rows > 48) gemm_pass<GATE_UP, 4>(c, st0, st1, st2, st3, bias_s, du.m0, du.rows);
  else if (du.rows > 32) gemm_pass<GATE_UP, 3>(c, st0, st1, st2, st3, bias_s, du.m0, du.rows);
  else gemm_pass<GATE_UP, 2>(c, st0, st1, st2, st3, bias_s, du.m0, du.rows);
}

// ---- dense groups on the scaled MFMA: fp8 activations x MXFP4 weights -------------------------------
// v_mfma_scale_f32_16x16x128_f8f6f4 takes A = 16 activation rows x 128 K as fp8 e4m3 and B = 128 K x 16
// weight rows as fp4 e2m1.  Measured on gfx950 (one-hot operands): an fp4 B lane (r, g) holds the 32
// K values 32g .. 32g+31 of its row r; an fp8 A lane (r, g) holds K 16g .. 16g+15 in bytes 0..15 and
// K 64+16g .. 64+16g+15 in bytes 16..31; and the E8M0 scale of 32-block b (K 32b .. 32b+31) is the
// scale byte of lane group b, for A and B alike, whichever lanes hold the block's values.  The packed
// MXFP4 tiles already hold exactly B's lane layout (lane 16g + r = row r, block 4kg + g of group kg,
// 16 bytes) and the block scales of the format, so the weights go from the load straight into the
// MFMA: no conversion and no scaling instruction.  The
// activations are quantised once per row to fp8 with one power-of-two scale per 32 values
// (mx_act_quant_kernel), whose scale bytes are stored in the same order as the weights': dword
// (kg4, g) of a row holds the scales of blocks 4(4kg4 + i) + g in bytes i = 0..3, so lane (r, g)
// finds the scale of its block of group kg in byte kg % 4 of one dword per 4 groups.  One MFMA covers
// what four bf16 MFMAs and eight conversions covered, and the activation stages carry half the bytes.
typedef int mx_v8i_t __attribute__((ext_vector_type(8)));

// bytes of one row's activation scales: 16 per 4 groups of 128 K (blocks past K read 127 = 2^0)
__host__ __device__ inline int mx_act_scale_row_bytes(int K) { return 16 * mx_geom(1, 16, K).KG4; }

// One wave per (row, 4 groups of 128 K): 8 elements per lane from one 16-byte load, 4 lanes per
// 32-block.  Each row is carried as two e4m3 terms, x = s1 q1 + s2 q2 + (rounding of the second term):
// the high term per block is s1 = 2^ceil(log2(max(amax, 1e-4) / 448)) (amax by xor shuffles), q1 = e4m3
// RNE of clamp(x / s1, +-448) (v_cvt_pk_fp8_f32); the residual x - s1 q1 is exact in fp32 (q1 s1 is x
// rounded to 4 significant bits), and the low term is the same rule applied to it.  Together they hold
// the 8 significant bits of a bf16 x, so the scaled-MFMA products carry the bf16 operand's precision.
// Row r's high term is row r of q and s, its low term row M + r.  Scale byte e + 127; blocks past K (up
// to 16 * KG4 per row) only write their scale byte, 127.
__device__ __forceinline__ int mx_block_scale_exp(float amax) {
  amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
  amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
  amax = fmaxf(amax, 1e-4f);
  // ceil(log2(amax / 448)) from the bits of amax * (1/448), a normal number since amax >= 1e-4
  const uint32_t bits = __float_as_uint(amax * (1.0f / 448.0f));
  return (int)((bits >> 23) & 0xff) - 127 + ((bits & 0x7fffffu) ? 1 : 0);
}

// e4m3 bytes of v * 2^-e (clamped to +-448), two dwords; dec receives the values the bytes hold
__device__ __forceinline__ uint2 mx_fp8_pack(const float (&v)[8], int e, float (&dec)[8]) {
  uint32_t w[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    float y[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) y[j] = fminf(fmaxf(ldexpf(v[4 * i + j], -e), -448.0f), 448.0f);
    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false);
    w[i] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], lo, true);
    dec[4 * i + 0] = __builtin_amdgcn_cvt_f32_fp8((int)w[i], 0);
    dec[4 * i + 1] = __builtin_amdgcn_cvt_f32_fp8((int)w[i], 1);
    dec[4 * i + 2] = __builtin_amdgcn_cvt_f32_fp8((int)w[i], 2);
    dec[4 * i + 3] = __builtin_amdgcn_cvt_f32_fp8((int)w[i], 3);
  }
  return make_uint2(w[0], w[1]);
}

__global__ __launch_bounds__(256) void mx_act_quant_kernel(const uint16_t* __restrict__ x, int M, int K,
                                                           uint8_t* __restrict__ q, uint8_t* __restrict__ s) {
  const MxGeom gm = mx_geom(1, 16, K);
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= M * gm.KG4) return;  // uniform per wave
  const int lane = threadIdx.x & 63;
  const int row = item / gm.KG4, kg4 = item % gm.KG4;
  const int k0 = kg4 * 512 + 8 * lane;
  const bool in = k0 < K;  // K % 32 == 0: a 32-block (4 lanes) is wholly inside or wholly past the row
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 xv = in ? *reinterpret_cast<const u32x4*>(x + (size_t)row * K + k0) : u32x4{0u, 0u, 0u, 0u};
  float v[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = bf2f(xv[i] & 0xffff);
    v[2 * i + 1] = bf2f(xv[i] >> 16);
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  const int e1 = mx_block_scale_exp(amax);
  float d1[8], r[8], d2[8];
  const uint2 w1 = mx_fp8_pack(v, e1, d1);
  float ramax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    r[i] = v[i] - ldexpf(d1[i], e1);  // exact: the high term is v rounded to 4 significant bits
    ramax = fmaxf(ramax, fabsf(r[i]));
  }
  const int e2 = mx_block_scale_exp(ramax);
  const uint2 w2 = mx_fp8_pack(r, e2, d2);
  if (in) {
    *reinterpret_cast<uint2*>(q + (size_t)row * K + k0) = w1;
    *reinterpret_cast<uint2*>(q + (size_t)(M + row) * K + k0) = w2;
  }
  if ((lane & 3) == 0) {
    const int blk = kg4 * 16 + lane / 4;  // block index within the row
    const int kg = blk / 4, g = blk % 4;
    const size_t at = ((kg >> 2) * 4 + g) * 4 + (kg & 3);
    const size_t rb = mx_act_scale_row_bytes(K);
    s[(size_t)row * rb + at] = in ? (uint8_t)(e1 + 127) : 127;
    s[(size_t)(M + row) * rb + at] = in ? (uint8_t)(e2 + 127) : 127;
  }
}

constexpr int kMxMaxMT = 12;  // row tiles per pass: up to 6 real row tiles, each as a high and a low tile
constexpr int kMxStage = kMxMaxMT * 2048 + kMxMaxMT * 256 + kGemmTiles * 256;  // activations, their scales, weight scales

// what one workgroup of the scaled GEMM works on
struct MxCtx {
  const uint8_t* act;     // fp8 activation rows [*, K]: high terms, then low terms from row lo_off
  const uint8_t* ascale;  // their scale rows, mx_act_scale_row_bytes(K) each
  const int32_t* perm;
  const float* bias;
  void* out;
  const uint8_t* wbase;  // the expert's packed tiles, + lane * 16
  const uint8_t* sbase;  // the expert's weight scale rows, + lane * 4
  MxGeom gm;
  size_t tile_bytes;
  int as_row, k_top, N, K, e, nb0, nbn, row_lo, lo_off, lane, wave, r, g;
};

// One pass over MT row tiles (16 * MT rows from m0) and every weight block of the chunk.  The pipeline
// is the bf16 dense kernel's: per group of 128 K, each wave loads its 2 weight tiles into a 4-deep
// register ring and DMAs its share of the activation fragments, their scale dwords and its tiles'
// scale dwords into one of 4 LDS stages, 3 groups ahead; a stage is waited for with an explicit vmcnt
// that leaves the 2 younger groups in flight, then a bare s_barrier.  The activation stage holds, for
// row tile m, two 1-KiB blocks (h = 0, 1): lane (g, r) at 16 * lane has bytes 64h + 16g .. +15 of the
// group of row 16m + r (the A operand's lane layout above), so a lane's A operand is two contiguous,
// conflict-free ds_read_b128.
template <bool GATE_UP, int MT>
__device__ __forceinline__ void mx_gemm_pass(const MxCtx& c, char (&st0)[kMxStage], char (&st1)[kMxStage],
                                             char (&st2)[kMxStage], char (&st3)[kMxStage],
                                             float (&bias_s)[kGemmBiasBlocks * 256], int m0, int rows) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) void* lds_ptr;
  static_assert(MT == 4 || MT == 8 || MT == 12, "row tiles per pass");
  constexpr int MR = MT / 2;                   // real row tiles: tile m < MR is the high term, m + MR the low
  constexpr int ASOFF = MT * 2048;             // activation scale dwords: MT x 256 B
  constexpr int WSOFF = ASOFF + MT * 256;      // weight scale dwords: 16 tiles x 256 B
  constexpr int AJ = MT / 4;                   // activation fragment blocks per wave per group
  constexpr int SJ = (MT + 7) / 8;             // activation scale blocks per wave per group
  constexpr int LOADS = 2 + 2 + AJ + SJ;       // weight tiles, weight scales, activations, their scales
  constexpr int WAIT = (kGemmStages - 2) * LOADS;
  const MxGeom& gm = c.gm;
  const int lane = c.lane, wave = c.wave, r = c.r, g = c.g;
  auto tile_of = [&](int nb, int n) __attribute__((always_inline)) {
    return min((c.nb0 + nb) * kGemmTiles + 2 * wave + n, gm.NT - 1);
  };
  // activation row of lane r of row tile t (t >= MR: the low term of tile t - MR)
  auto src_row = [&](int t) __attribute__((always_inline)) {
    const int row = (t % MR) * 16 + r;
    const int p = c.row_lo + m0 + (row < rows ? row : 0);  // rows past the pass read row 0, never stored
    return (GATE_UP ? c.perm[p] / c.k_top : p) + (t >= MR ? c.lo_off : 0);
  };
  const int KGP = (gm.KG + kGemmStages - 1) / kGemmStages * kGemmStages;  // groups per block, padded
  // DMA sources: fragment block b = J*8 + wave is row tile b/2, half b%2; scale blocks wave + 8 j
  // (clamped: waves past the last tile load a copy of an earlier one, so every wave issues SJ loads)
  const uint8_t* arow[AJ];
  int akl[AJ];  // the lane's K offset within a group, for the half its block holds
#pragma unroll
  for (int J = 0; J < AJ; ++J) {
    const int b = J * 8 + wave;
    akl[J] = 64 * (b & 1) + 16 * g;
    arow[J] = c.act + (size_t)src_row(b >> 1) * c.K + akl[J];
  }
  const uint8_t* asrow[SJ];
  int astile[SJ];
#pragma unroll
  for (int j = 0; j < SJ; ++j) {
    astile[j] = (wave + 8 * j) < MT ? wave + 8 * j : wave % MT;
    asrow[j] = c.ascale + (size_t)src_row(astile[j]) * c.as_row + 4 * g;
  }
  int i_nb = 0, i_kg = 0;
  auto issue = [&](u32x4 (&bq)[2], char* stage) __attribute__((always_inline)) {
    const int nb = min(i_nb, c.nbn - 1), kg = i_kg;
    const bool blk = 4 * kg + g < gm.G;  // the lane's block of the group exists
    const size_t woff = blk ? (size_t)kg * 1024 : 0;
#pragma unroll
    for (int n = 0; n < 2; ++n)
      bq[n] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(c.wbase + (size_t)tile_of(nb, n) * c.tile_bytes + woff));
#pragma unroll
    for (int n = 0; n < 2; ++n)
      __builtin_amdgcn_global_load_lds((const void*)(c.sbase + ((size_t)tile_of(nb, n) * gm.KG4 + min(kg / 4, gm.KG4 - 1)) * 256),
                                       (lds_ptr)(stage + WSOFF + (2 * wave + n) * 256), 4, 0, 0);
    // lanes whose 16 K values lie past the row read its first group instead (finite, and paired with
    // zeroed weights)
#pragma unroll
    for (int J = 0; J < AJ; ++J)
      __builtin_amdgcn_global_load_lds((const void*)(arow[J] + (kg * 128 + akl[J] < c.K ? kg * 128 : 0)),
                                       (lds_ptr)(stage + (J * 8 + wave) * 1024), 16, 0, 0);
#pragma unroll
    for (int j = 0; j < SJ; ++j)
      __builtin_amdgcn_global_load_lds((const void*)(asrow[j] + min(kg / 4, gm.KG4 - 1) * 16),
                                       (lds_ptr)(stage + ASOFF + astile[j] * 256), 4, 0, 0);
    if (++i_kg == KGP) {
      i_kg = 0;
      ++i_nb;
    }
  };
  f32x4_t acc[MT][2];
  auto zero_acc = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int n = 0; n < 2; ++n) acc[m][n] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  };
  zero_acc();
  u32x4 w0[2], w1[2], w2[2], w3[2];
  // group kg from stage `cur` and weight slot `wq`: A fragments and scales from LDS, B straight from
  // the ring (lanes past the row's last block zeroed), MT x 2 scaled MFMAs
  auto compute = [&](const char* cur, const u32x4 (&wq)[2], int kg) __attribute__((always_inline)) {
    const int sh = 8 * (kg & 3);
    const bool bok = 4 * kg + g < gm.G;
    int sw[2];
    mx_v8i_t b[2];
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      sw[n] = (int)((*reinterpret_cast<const uint32_t*>(cur + WSOFF + (2 * wave + n) * 256 + lane * 4) >> sh) & 0xffu);
      const u32x4 wv = bok ? wq[n] : u32x4{0u, 0u, 0u, 0u};
      b[n] = mx_v8i_t{(int)wv.x, (int)wv.y, (int)wv.z, (int)wv.w, 0, 0, 0, 0};
    }
    // row tile m's operand is read while tile m-1's two MFMAs run (two operand sets live, not MT)
    u32x4 lo[2], hi[2];
    uint32_t sdw[2];
    auto read_a = [&](auto m) __attribute__((always_inline)) {
      constexpr int q = decltype(m)::value & 1;
      lo[q] = *reinterpret_cast<const u32x4*>(cur + (2 * m) * 1024 + lane * 16);
      hi[q] = *reinterpret_cast<const u32x4*>(cur + (2 * m + 1) * 1024 + lane * 16);
      sdw[q] = *reinterpret_cast<const uint32_t*>(cur + ASOFF + m * 256 + lane * 4);
    };
    read_a(std::integral_constant<int, 0>{});
    mx_static_for<0, MT>([&](auto m) {
      constexpr int q = decltype(m)::value & 1;
      if constexpr (decltype(m)::value + 1 < MT) read_a(std::integral_constant<int, decltype(m)::value + 1>{});
      const int sa = (int)((sdw[q] >> sh) & 0xffu);
      const mx_v8i_t a = mx_v8i_t{(int)lo[q].x, (int)lo[q].y, (int)lo[q].z, (int)lo[q].w,
                                  (int)hi[q].x, (int)hi[q].y, (int)hi[q].z, (int)hi[q].w};
#pragma unroll
      for (int n = 0; n < 2; ++n)
        acc[m][n] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b[n], acc[m][n], 0, 4, 0, sa, 0, sw[n]);
    });
    // the order above, kept by the scheduler: weight scales and tile 0's reads, then per tile the next
    // tile's 3 reads and this tile's 2 MFMAs
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 5, 0);
    mx_static_for<0, MT - 1>([&](auto) {
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 3, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 0);
    });
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 0);
    __builtin_amdgcn_sched_barrier(0);
  };
  float bsum[2];
  auto load_bias = [&](int nb) __attribute__((always_inline)) {
#pragma unroll
    for (int n = 0; n < 2; ++n) bsum[n] = bias_s[(tile_of(min(nb, c.nbn - 1), n) - c.nb0 * kGemmTiles) * 16 + r];
  };
  // acc[m][n][v] = D[group row 16m + 4g + v][feature (block tile 2*wave + n) * 16 + r] of the high term
  // (m < MR) or the low term (m >= MR, row 16(m - MR) + 4g + v)
  auto epilogue = [&](int nb) __attribute__((always_inline)) {
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      const int tile = (c.nb0 + nb) * kGemmTiles + 2 * wave + n;
      const bool nval = tile < gm.NT;
      const int feat = tile * 16 + r;
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        float val[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) val[v] = (acc[m][n][v] + acc[m + MR][n][v]) + bsum[n];
        if (GATE_UP) {
          swiglu_pairs(val, r, [&](int v, uint16_t hbits) {
            const int orow = 16 * m + 4 * g + v;
            if (nval && orow < rows)
              reinterpret_cast<uint16_t*>(c.out)[(size_t)(c.row_lo + m0 + orow) * (c.N / 2) + feat / 2] = hbits;
          });
        } else {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int orow = 16 * m + 4 * g + v;
            if (nval && orow < rows)
              reinterpret_cast<float*>(c.out)[(size_t)(c.row_lo + m0 + orow) * c.N + feat] = val[v];
          }
        }
      }
    }
  };
  auto group = [&](char* cur, u32x4 (&wq)[2], int kg) __attribute__((always_inline)) {
    compute(cur, wq, kg);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(WAIT));  // this wave's loads of the next group are done
    lds_barrier();  // every wave's part of the next stage is in LDS; every wave is done with `cur`
    issue(wq, cur);  // refill `cur` and the weight slot 4 groups ahead
  };

  lds_barrier();  // every wave is done with the previous pass's stages (and the bias)
  stage_chunk_bias(c.bias, c.e, c.N, c.nb0, c.nbn, bias_s);
  // the stage waits count loads per group in issue order: no load may move across a group
  asm volatile("" ::: "memory");
  issue(w0, st0);
  asm volatile("" ::: "memory");
  issue(w1, st1);
  asm volatile("" ::: "memory");
  issue(w2, st2);
  asm volatile("" ::: "memory");
  issue(w3, st3);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(waitcnt_vm((kGemmStages - 1) * LOADS));
  lds_barrier();  // stage 0 is in LDS
  for (int nb = 0; nb < c.nbn; ++nb) {
    for (int kg = 0; kg < KGP; kg += kGemmStages) {
      group(st0, w0, kg);
      group(st1, w1, kg + 1);
      group(st2, w2, kg + 2);
      group(st3, w3, kg + 3);
    }
    load_bias(nb);
    epilogue(nb);
    zero_acc();
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // the loads past the chunk's end have landed
}

template <bool GATE_UP>
__global__ __launch_bounds__(512) void moe_mx_gemm_kernel(
    const uint8_t* __restrict__ act, const uint8_t* __restrict__ ascale, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ offsets, int k_top, const uint8_t* __restrict__ packed,
    const float* __restrict__ bias, int E, int N, int K, int min_rows, int chunk, int lo_off,
    void* __restrict__ out) {
  __shared__ __align__(16) char st0[kMxStage];
  __shared__ __align__(16) char st1[kMxStage];
  __shared__ __align__(16) char st2[kMxStage];
  __shared__ __align__(16) char st3[kMxStage];
  MxCtx c;
  c.gm = mx_geom(E, N, K);
  const int blocks_per_e = (c.gm.NT + kGemmTiles - 1) / kGemmTiles;
  const int chunks_per_e = (blocks_per_e + chunk - 1) / chunk;
  __shared__ int pass_pre[257];
  __shared__ float bias_s[kGemmBiasBlocks * 256];
  DenseUnit du;
  int unit = 0;
  if (!dense_unit(offsets, E, min_rows, chunks_per_e, pass_pre, du, unit)) return;
  c.e = du.e;
  c.nb0 = (unit % chunks_per_e) * chunk;
  c.nbn = min(chunk, blocks_per_e - c.nb0);
  c.row_lo = du.row_lo;
  c.act = act;
  c.ascale = ascale;
  c.perm = perm;
  c.bias = bias;
  c.out = out;
  c.k_top = k_top;
  c.N = N;
  c.K = K;
  c.as_row = mx_act_scale_row_bytes(K);
  c.lo_off = lo_off;
  const int tid = threadIdx.x;
  c.lane = tid & 63;
  c.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  c.r = c.lane & 15;
  c.g = c.lane >> 4;
  c.tile_bytes = (size_t)c.gm.G * 256;
  c.wbase = packed + (size_t)c.e * c.gm.NT * c.tile_bytes + c.lane * 16;
  c.sbase = packed + c.gm.data_bytes + (size_t)c.e * c.gm.NT * c.gm.KG4 * 256 + c.lane * 4;
  // this unit's pass of 96 rows (6 row tiles, each with its high and low term); a group's last pass takes
  // the fewest 32-row multiples that hold its rows
  if (du.rows > 64) mx_gemm_pass<GATE_UP, 12>(c, st0, st1, st2, st3, bias_s, du.m0, du.rows);
  else if (du.rows > 32) mx_gemm_pass<GATE_UP, 8>(c, st0, st1, st2, st3, bias_s, du.m0, du.rows);
  else mx_gemm_pass<GATE_UP, 4>(c, st0, st1, st2, st3, bias_s, du.m0, du.rows);
}

// Chunk of weight blocks per workgroup: the largest chunk that still gives at least 3 rounds of
// workgroups over the CUs, so that workgroups of unequal length (experts with different row
// counts take different row tiles) balance, while each start-up is shared by several blocks.
// The CU count is read per device (once each) for the device current at the call.
inline int device_cus() {
  constexpr int kDevices = 64;
  static std::atomic<int> cached[kDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kDevices) return 256;
  int v = cached[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
  cached[dev].store(v, std::memory_order_relaxed);
  return v;
}

inline int gemm_chunk(const MxGeom& gm, int E) {
  const int cus = device_cus();
  const int W = (gm.NT + kGemmTiles - 1) / kGemmTiles;
  int best = 1;
  for (int c = 1; c <= min(W, kGemmBiasBlocks); ++c)
    if ((int64_t)E * ((W + c - 1) / c) >= 3LL * cus) best = c;
  return best;
}

// grid of the tiled GEMM: the work units (expert, chunk of weight blocks) rounded up to 8 XCDs
inline int gemm_grid(const MxGeom& gm, int E, int chunk, int rows_total) {
  const int W = (gm.NT + kGemmTiles - 1) / kGemmTiles;
  const int units = (E + ceil_div(rows_total, kGemmRows)) * ((W + chunk - 1) / chunk);
  return ((units + 7) / 8) * 8;
}

// Groups of more than kDenseFrom rows take the dense kernel when the batch averages at least that
// many rows per expert (otherwise the row-pass kernel serves every group: a rare large group costs
// extra passes, not a launch of mostly idle workgroups).  Both kernels are correct for any count.
constexpr int kDenseFrom = 8;

inline bool use_dense(int rows_total, int E) { return (int64_t)rows_total >= (int64_t)kDenseFrom * E; }

// whether a batch of rows_total permuted rows gives any expert group to the dense kernels
bool moe_batch_is_dense(int rows_total, int E, int K) { return use_dense(rows_total, E) && K >= 128; }

int launch_moe_gate_up(const uint16_t* x, const int32_t* perm, const int32_t* offsets, int k_top,
                       const uint8_t* w13, const float* b13, int T, int E, int H, int I, uint16_t* h,
                       hipStream_t s) {
  const MxGeom gm = mx_geom(E, 2 * I, H);
  const bool dense = use_dense(T * k_top, E) && H >= 128;  // the tiled kernel reads 128-K groups
  if (H <= 4064) {
    const int wg_per_e = ceil_div(gm.NT, 4 * kNTWGateUp);
    hipLaunchKernelGGL((moe_mxfp4_kernel<true, kNTWGateUp, kDepthGateUp>), dim3(E * wg_per_e), dim3(256),
                       kRowsPerPass * mx_lds_row_bytes(H), s, x, perm, offsets, k_top, w13, b13, E,
                       2 * I, H, 1, dense ? kDenseFrom : (1 << 30), (void*)h);
    int rc = check_launch("moe_gate_up_mxfp4");
    if (rc) return rc;
  }
  if (dense || H > 4064) {
    const int chunk = gemm_chunk(gm, E);
    hipLaunchKernelGGL((moe_mxfp4_gemm_kernel<true>), dim3(gemm_grid(gm, E, chunk, T * k_top)), dim3(512), 0, s,
                       x, perm, offsets, k_top, w13, b13, E, 2 * I, H, H > 4064 ? 1 : kDenseFrom + 1, chunk,
                       (void*)h);
    return check_launch("moe_gate_up_mxfp4(dense)");
  }
  return FLYAI_OK;
}

int launch_moe_down(const uint16_t* h, const int32_t* offsets, const uint8_t* w2, const float* b2,
                    int rows_total, int E, int H, int I, float* y, hipStream_t s) {
  const MxGeom gm = mx_geom(E, H, I);
  const bool dense = use_dense(rows_total, E) && I >= 128;  // the tiled kernel reads 128-K groups
  if (I <= 4064) {
    const int wg_per_e = ceil_div(gm.NT, 4 * kNTWDown);
    hipLaunchKernelGGL((moe_mxfp4_kernel<false, kNTWDown, kDepthDown>), dim3(E * wg_per_e), dim3(256),
                       kRowsPerPass * mx_lds_row_bytes(I), s, h, nullptr, offsets, 1, w2, b2, E, H, I, 1,
                       dense ? kDenseFrom : (1 << 30), (void*)y);
    int rc = check_launch("moe_down_mxfp4");
    if (rc) return rc;
  }
  if (dense || I > 4064) {
    const int chunk = gemm_chunk(gm, E);
    hipLaunchKernelGGL((moe_mxfp4_gemm_kernel<false>), dim3(gemm_grid(gm, E, chunk, rows_total)), dim3(512), 0, s,
                       h, nullptr, offsets, 1, w2, b2, E, H, I, I > 4064 ? 1 : kDenseFrom + 1, chunk, (void*)y);
    return check_launch("moe_down_mxfp4(dense)");
  }
  return FLYAI_OK;
}

int launch_mx_act_quant(const uint16_t* x, int M, int K, uint8_t* q, uint8_t* s, hipStream_t st) {
  if (M == 0) return FLYAI_OK;
  const int items = M * mx_geom(1, 16, K).KG4;
  hipLaunchKernelGGL(mx_act_quant_kernel, dim3(ceil_div(items, 4)), dim3(256), 0, st, x, M, K, q, s);
  return check_launch("mx_act_quant");
}

// The fp8-activation variants: groups the bf16 kernels would give the dense tiled GEMM take the
// scaled-MFMA GEMM on the quantised rows instead; decode-sized groups keep the row-pass kernel on the
// bf16 rows.
int launch_moe_gate_up_fp8act(const uint16_t* x, const uint8_t* xq, const uint8_t* xs, const int32_t* perm,
                              const int32_t* offsets, int k_top, const uint8_t* w13, const float* b13, int T,
                              int E, int H, int I, uint16_t* h, hipStream_t s) {
  const MxGeom gm = mx_geom(E, 2 * I, H);
  const bool dense = use_dense(T * k_top, E) && H >= 128;
  if (H <= 4064) {
    const int wg_per_e = ceil_div(gm.NT, 4 * kNTWGateUp);
    hipLaunchKernelGGL((moe_mxfp4_kernel<true, kNTWGateUp, kDepthGateUp>), dim3(E * wg_per_e), dim3(256),
                       kRowsPerPass * mx_lds_row_bytes(H), s, x, perm, offsets, k_top, w13, b13, E,
                       2 * I, H, 1, dense ? kDenseFrom : (1 << 30), (void*)h);
    const int rc = check_launch("moe_gate_up_mxfp4");
    if (rc) return rc;
  }
  if (dense || H > 4064) {
    const int chunk = gemm_chunk(gm, E);
    hipLaunchKernelGGL((moe_mx_gemm_kernel<true>), dim3(gemm_grid(gm, E, chunk, T * k_top)), dim3(512), 0, s, xq, xs, perm,
                       offsets, k_top, w13, b13, E, 2 * I, H, H > 4064 ? 1 : kDenseFrom + 1, chunk, T, (void*)h);
    return check_launch("moe_gate_up_mxfp4(scaled mfma)");
  }
  return FLYAI_OK;
}

int launch_moe_down_fp8act(const uint16_t* h, const uint8_t* hq, const uint8_t* hs, const int32_t* offsets,
                           const uint8_t* w2, const float* b2, int rows_total, int E, int H, int I, float* y,
                           hipStream_t s) {
  const MxGeom gm = mx_geom(E, H, I);
  const bool dense = use_dense(rows_total, E) && I >= 128;
  if (I <= 4064) {
    const int wg_per_e = ceil_div(gm.NT, 4 * kNTWDown);
    hipLaunchKernelGGL((moe_mxfp4_kernel<false, kNTWDown, kDepthDown>), dim3(E * wg_per_e), dim3(256),
                       kRowsPerPass * mx_lds_row_bytes(I), s, h, nullptr, offsets, 1, w2, b2, E, H, I, 1,
                       dense ? kDenseFrom : (1 << 30), (void*)y);
    const int rc = check_launch("moe_down_mxfp4");
    if (rc) return rc;
  }
  if (dense || I > 4064) {
    const int chunk = gemm_chunk(gm, E);
    hipLaunchKernelGGL((moe_mx_gemm_kernel<false>), dim3(gemm_grid(gm, E, chunk, rows_total)), dim3(512), 0, s, hq, hs, nullptr,
                       offsets, 1, w2, b2, E, H, I, I > 4064 ? 1 : kDenseFrom + 1, chunk, rows_total, (void*)y);
    return check_launch("moe_down_mxfp4(scaled mfma)");
  }
  return FLYAI_OK;
}

}  // namespace flyai

using namespace flyai;

extern "C" size_t flyai_mxfp4_packed_bytes(int32_t E, int32_t N, int32_t K) {
  if (E <= 0 || N <= 0 || K <= 0 || N % 16 || K % 32) return 0;
  const MxGeom g = mx_geom(E, N, K);
  return g.data_bytes + (size_t)E * g.NT * g.KG4 * 256;
}

extern "C" int flyai_mxfp4_repack(const uint8_t* blocks, const uint8_t* scales, int32_t E, int32_t N,
                                  int32_t K, uint8_t* packed, flyai_stream_t stream) {
  FLYAI_REQUIRE(E > 0 && N > 0 && K > 0 && N % 16 == 0 && K % 32 == 0,
                "repack: need N %% 16 == 0 and K %% 32 == 0");
  FLYAI_REQUIRE(blocks && scales && packed, "repack: null pointer");
  const MxGeom gm = mx_geom(E, N, K);
  const size_t total = (size_t)E * gm.NT * gm.KG * 64;
  hipLaunchKernelGGL(mxfp4_repack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     as_stream(stream), blocks, scales, E, N, K, packed);
  return check_launch("mxfp4_repack");
}

extern "C" int flyai_moe_gate_up_mxfp4(const uint16_t* x, const int32_t* perm,
                                       const int32_t* offsets, int32_t T, int32_t k,
                                       const uint8_t* w13_packed, const float* b13, int32_t E,
                                       int32_t H, int32_t I, uint16_t* h, flyai_stream_t stream) {
  FLYAI_REQUIRE(T >= 0 && E > 0 && E <= 256 && H > 0 && I > 0 && H % 32 == 0 && (2 * I) % 16 == 0 && k >= 1,
                "gate_up: need 1 <= E <= 256, H %% 32 == 0, 2I %% 16 == 0");
  FLYAI_REQUIRE(x && perm && offsets && w13_packed && b13 && h, "gate_up: null pointer");
  return launch_moe_gate_up(x, perm, offsets, k, w13_packed, b13, T, E, H, I, h, as_stream(stream));
}

extern "C" int flyai_moe_down_mxfp4(const uint16_t* h, const int32_t* offsets, int32_t rows,
                                    const uint8_t* w2_packed, const float* b2, int32_t E, int32_t H,
                                    int32_t I, float* y_perm, flyai_stream_t stream) {
  FLYAI_REQUIRE(rows >= 0 && E > 0 && E <= 256 && H > 0 && I > 0 && I % 32 == 0 && H % 16 == 0,
                "down: need 1 <= E <= 256, I %% 32 == 0, H %% 16 == 0");
  FLYAI_REQUIRE(h && offsets && w2_packed && b2 && y_perm, "down: null pointer");
  return launch_moe_down(h, offsets, w2_packed, b2, rows, E, H, I, y_perm, as_stream(stream));
}

extern "C" size_t flyai_mx_act_scale_bytes(int32_t M, int32_t K) {
  if (M < 0 || K <= 0 || K % 32) return 0;
  return (size_t)M * mx_act_scale_row_bytes(K);
}

extern "C" int flyai_mx_act_quant(const uint16_t* x, int32_t M, int32_t K, uint8_t* q, uint8_t* s,
                                  flyai_stream_t stream) {
  FLYAI_REQUIRE(M >= 0 && K > 0 && K % 32 == 0, "mx_act_quant: need K %% 32 == 0");
  FLYAI_REQUIRE(x && q && s, "mx_act_quant: null pointer");
  return launch_mx_act_quant(x, M, K, q, s, as_stream(stream));
}

extern "C" int flyai_moe_gate_up_mxfp4_fp8act(const uint16_t* x, const uint8_t* xq, const uint8_t* xs,
                                              const int32_t* perm, const int32_t* offsets, int32_t T, int32_t k,
                                              const uint8_t* w13_packed, const float* b13, int32_t E, int32_t H,
                                              int32_t I, uint16_t* h, flyai_stream_t stream) {
  FLYAI_REQUIRE(T >= 0 && E > 0 && E <= 256 && H > 0 && I > 0 && H % 32 == 0 && (2 * I) % 16 == 0 && k >= 1,
                "gate_up: need 1 <= E <= 256, H %% 32 == 0, 2I %% 16 == 0");
  FLYAI_REQUIRE(x && xq && xs && perm && offsets && w13_packed && b13 && h, "gate_up: null pointer");
  return launch_moe_gate_up_fp8act(x, xq, xs, perm, offsets, k, w13_packed, b13, T, E, H, I, h, as_stream(stream));
}

extern "C" int flyai_moe_down_mxfp4_fp8act(const uint16_t* h, const uint8_t* hq, const uint8_t* hs,
                                           const int32_t* offsets, int32_t rows, const uint8_t* w2_packed,
                                           const float* b2, int32_t E, int32_t H, int32_t I, float* y_perm,
                                           flyai_stream_t stream) {
  FLYAI_REQUIRE(rows >= 0 && E > 0 && E <= 256 && H > 0 && I > 0 && I % 32 == 0 && H % 16 == 0,
                "down: need 1 <= E <= 256, I %% 32 == 0, H %% 16 == 0");
  FLYAI_REQUIRE(h && hq && hs && offsets && w2_packed && b2 && y_perm, "down: null pointer");
  return launch_moe_down_fp8act(h, hq, hs, offsets, w2_packed, b2, rows, E, H, I, y_perm, as_stream(stream));
}
