// gemm_i8.hip — int8 GEMM on gfx950 i8 MFMA (v_mfma_i32_32x32x32_i8) with
// exact int32 accumulation and the reference's dequantisation fused into
// the epilogue.
//
// Replaces linalg.MatMul8N (linalg/int8.go:89-155) and its VNNI tiles
// (kernel_vnni_amd64.s:13-256). The reference multiplies uint8 activations
// q+128 by int8 weights; MFMA is signed x signed, so the kernel sums q*w and
// rebuilds the reference tile exactly as acc + 128*colsum[n] (int32), then
// rescales it with the same float32 operations in the same order:
// ((f32(tile) - zc[n]) * sb[n]) * sa[m] (+ C).
//
// Block tile (64*MI)x128, K step 64, 256 threads: 4 waves (2x2), each a
// (32*MI)x64 tile of MIx2 MFMA 32x32 blocks. A and B stream into an
// ST-stage LDS ring with direct-to-LDS loads (global_load_lds_dwordx4: a
// wave instruction fills 1 KB, 16 rows of 64 bytes); the 16-byte chunks of
// a row are XOR-swizzled by (row >> 1) & 3 so the 16-byte fragment reads of
// consecutive rows fall in distinct banks. One barrier per K step; loads
// run ST-1 K steps ahead. Tiles are handed out XCD by XCD so the N-tiles of
// an A panel share one L2. The default is 128x128 with 2 stages: 35 KB of
// LDS and ~100 VGPRs let 4 workgroups share a CU, so one workgroup's
// epilogue stores overlap the others' MFMA loops (on the encoder's shapes
// it beats 256x128 tiles by 8-22%).
#include <stdlib.h>

#include "ixh_device.h"
#include "ixh_internal.h"

namespace ixh {

namespace {

constexpr int BN = 128, BK = 64, NXCD = 8;
constexpr int EPI_TILE_BYTES = 4 * 32 * 68 * 4;  // epilogue LDS tiles of the 4 waves

// Tile configurations: MI 32-row MFMA blocks per wave (block tile BM = 64*MI
// rows x 128 columns) and ST stages in the LDS ring.
template <int MI, int ST>
struct Cfg {
  static constexpr int BM = 64 * MI, LOADS = MI + 2;  // direct-to-LDS loads per wave per stage
  static constexpr int A_BYTES = BM * BK, STAGE_BYTES = (BM + BN) * BK;
  static constexpr int SMEM = ST * STAGE_BYTES > EPI_TILE_BYTES ? ST * STAGE_BYTES : EPI_TILE_BYTES;
};

// wait until at most `stages` later stages (of L loads each) are in flight
template <int L>
__device__ __forceinline__ void wait_stages(int stages) {
  if (stages >= 2)
    wait_vmcnt<2 * L>();
  else if (stages == 1)
    wait_vmcnt<L>();
  else
    wait_vmcnt<0>();
}

template <int EPI, int MI, int ST>
__global__ __launch_bounds__(256, MI == 4 ? 2 : 3) void gemm_i8_kernel(GemmArgs a) {
  using C = Cfg<MI, ST>;
  constexpr int BM = C::BM, A_BYTES = C::A_BYTES, STAGE_BYTES = C::STAGE_BYTES;
  extern __shared__ __attribute__((aligned(1024))) int8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int ntn = a.Np / BN, ntm = (a.M + BM - 1) / BM;
  const int tiles = ntm * ntn;
  // XCD-aware order: block b runs on XCD b % 8; give each XCD a contiguous
  // run of tiles, N fastest.
  const int per_xcd = (tiles + NXCD - 1) / NXCD;
  const int tix = (blockIdx.x % NXCD) * per_xcd + blockIdx.x / NXCD;
  if (tix >= tiles) return;
  const int nt = tix % ntn, mt = tix / ntn;
  const int m0 = mt * BM, n0 = nt * BN;

  // This wave's direct-to-LDS loads of a stage: A chunks MI*wave..+MI-1
  // (rows 16*MI*wave + 16u + lane/4), B chunks 2*wave..+1 (rows 32*wave +
  // 16u + lane/4). Lane i fills LDS bytes 16i of its chunk: row i/4,
  // physical 16-byte column i%4, i.e. logical column (i%4) ^ swz(row).
  const int lrow = lane >> 2, lchunk = (lane & 3) ^ swz(lane >> 2);
  glb_ptr ag[MI];
  glb_ptr bg[2];
#pragma unroll
  for (int u = 0; u < MI; u++) {
    int row = m0 + 16 * MI * wave + 16 * u + lrow;
    row = row < a.M ? row : a.M - 1;  // rows past M load row M-1 (never stored)
    ag[u] = (glb_ptr)(a.A + (size_t)row * a.lda + 16 * lchunk);
  }
#pragma unroll
  for (int u = 0; u < 2; u++)
    bg[u] = (glb_ptr)(a.B + (size_t)(n0 + 32 * wave + 16 * u + lrow) * a.ldb + 16 * lchunk);

  auto issue = [&](int kt) {
    int8_t *st = smem + (kt % ST) * STAGE_BYTES;
    const int k0 = kt * BK;
#pragma unroll
    for (int u = 0; u < MI; u++)
      __builtin_amdgcn_global_load_lds((glb_ptr)((const int8_t *)ag[u] + k0),
                                       (lds_ptr)(st + (16 * MI * wave + 16 * u) * BK), 16, 0, 0);
#pragma unroll
    for (int u = 0; u < 2; u++)
      __builtin_amdgcn_global_load_lds((glb_ptr)((const int8_t *)bg[u] + k0),
                                       (lds_ptr)(st + A_BYTES + (32 * wave + 16 * u) * BK), 16, 0, 0);
  };

  v16i acc[MI][2];
#pragma unroll
  for (int i = 0; i < MI; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0;

  // per-row activation scales of the tile, for the epilogue
  __shared__ float sa_s[BM];
  __shared__ int pos_s[EPI == EPI_ROPE ? BM : 1];
  if (tid < BM) {
    sa_s[tid] = a.sa[min(m0 + tid, a.M - 1)];
    if constexpr (EPI == EPI_ROPE) pos_s[tid] = a.pos[min(m0 + tid, a.M - 1)];
  }

  const int nk = a.Kp / BK;
  const int fr = lane & 31, fh = lane >> 5;
#pragma unroll
  for (int p = 0; p < ST - 1; p++)
    if (p < nk) issue(p);
  for (int kt = 0; kt < nk; kt++) {
    // this K step's loads done, the next ST-2 steps' may be in flight
    wait_stages<C::LOADS>(min(ST - 2, nk - 1 - kt));
    // every wave's loads landed; stage (kt+ST-1)%ST is free. A bare
    // s_barrier: __syncthreads' fence would also drain the next loads.
    __builtin_amdgcn_s_barrier();
    if (kt + ST - 1 < nk) issue(kt + ST - 1);
    const int8_t *st = smem + (kt % ST) * STAGE_BYTES;
#pragma unroll
    for (int s = 0; s < 2; s++) {
      v4i fa[MI], fb[2];
#pragma unroll
      for (int i = 0; i < MI; i++) {
        const int row = wm * 32 * MI + 32 * i + fr;
        fa[i] = *(const v4i *)(st + row * BK + 16 * ((2 * s + fh) ^ swz(row)));
      }
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int row = wn * 64 + 32 * j + fr;
        fb[j] = *(const v4i *)(st + A_BYTES + row * BK + 16 * ((2 * s + fh) ^ swz(row)));
      }
#pragma unroll
      for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = mfma32(fa[i], fb[j], acc[i][j]);
    }
  }

  // ---- epilogue ----
  // Values are formed in the MFMA layout (lane: column fr, 16 rows per
  // 32-row block), written to a per-wave LDS tile, and leave as 16-byte
  // row segments (the residual of EPI_ACCUM is read the same way).
  __syncthreads();  // the ring is no longer read: reuse it for the tiles
  const int nw = n0 + wn * 64;  // first column of the wave tile
  int ncol[2];
  float zc[2], sb[2];
  int c128[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    ncol[j] = nw + 32 * j + fr;
    zc[j] = a.zc[ncol[j]];
    sb[j] = a.sb[ncol[j]];
    c128[j] = a.c128[ncol[j]];
  }
  constexpr int LDT = 68;  // floats per LDS tile row (64 + 4 padding)
  float *tile = (float *)(smem + wave * (32 * LDT * 4));
  const bool vec = (a.ldc & 3) == 0;
#pragma unroll
  for (int i = 0; i < MI; i++) {
    const int rb = wm * 32 * MI + 32 * i;  // first row of the block in the tile
    // wave-uniform; a wave past M still meets both barriers below
    const bool live = m0 + rb < a.M;
    // RoPE tables of the block's 16 rows of this lane, gathered up front
    float rc[16], rs[16];
    if constexpr (EPI == EPI_ROPE) {
      if (live && nw < a.rope_cols) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int p = pos_s[rb + acc_row(r, lane)];
          rc[r] = a.rope_cos[(size_t)p * 32 + fr];
          rs[r] = a.rope_sin[(size_t)p * 32 + fr];
        }
      }
    }
    // (1) MFMA layout -> LDS tile
#pragma unroll
    for (int r = 0; r < 16 && live; r++) {
      const int rl = acc_row(r, lane);
      const int m = min(m0 + rb + rl, a.M - 1);
      const float sa = sa_s[rb + rl];
      if constexpr (EPI == EPI_TILE) {
        tile[rl * LDT + fr] = __int_as_float(acc[i][0][r] + c128[0]);
        tile[rl * LDT + 32 + fr] = __int_as_float(acc[i][1][r] + c128[1]);
      } else if constexpr (EPI == EPI_GEGLU) {
        // Columns nw..nw+31 hold the GELU input of gated columns
        // nw/2..nw/2+31, columns nw+32..nw+63 their multiplier
        // (Wi rows interleaved by 32 on upload; GeluMul vec_simd.go:125-160).
        const float va = deq(acc[i][0][r] + c128[0], zc[0], sb[0], sa);
        const float vb = deq(acc[i][1][r] + c128[1], zc[1], sb[1], sa);
        const int gc = nw / 2 + fr;
        const float ge = gc < a.n_gelu ? gelu_fma(va) : gelu_scalar(va);
        tile[rl * LDT + fr] = ge * vb;
      } else if constexpr (EPI == EPI_ROPE) {
        float v0 = deq(acc[i][0][r] + c128[0], zc[0], sb[0], sa);
        float v1 = deq(acc[i][1][r] + c128[1], zc[1], sb[1], sa);
        if (nw < a.rope_cols) {
          // linalg.Rope (vec_simd.go:408-425) on the head whose 64 values
          // are this wave tile: x1' = x1*c - x2*s, x2' = x2*c + x1*s.
          const float c = rc[r], s = rs[r];
          const float x1 = v0, x2 = v1;
          v0 = x1 * c - x2 * s;
          v1 = x2 * c + x1 * s;
        }
        if (nw < a.q_cols) {
          // the query head, quantised per row as Attn8.Prepare does
          // (attention8.go:211-220): the 64 values of the row are this
          // lane's two and those of the 31 other lanes of its half-wave.
          float mx = fmax32(fabsf(v0), fabsf(v1));
#pragma unroll
          for (int t = 1; t < 32; t <<= 1) mx = fmax32(mx, __shfl_xor(mx, t));
          float sc = 0.f, inv = 0.f;
          if (mx != 0.f) {
            sc = mx / 127.0f;
            inv = 1.0f / sc;
          }
          int8_t *qt = (int8_t *)tile;
          qt[rl * 64 + fr] = (int8_t)q8(v0, inv);
          qt[rl * 64 + 32 + fr] = (int8_t)q8(v1, inv);
          if (fr == 0 && m0 + rb + rl < a.M)
            a.sq[(size_t)(m0 + rb + rl) * (a.q_cols / 64) + nw / 64] = sc * a.attn_scale;
        } else {
          tile[rl * LDT + fr] = v0;
          tile[rl * LDT + 32 + fr] = v1;
        }
      } else {
        tile[rl * LDT + fr] = deq(acc[i][0][r] + c128[0], zc[0], sb[0], sa);
        tile[rl * LDT + 32 + fr] = deq(acc[i][1][r] + c128[1], zc[1], sb[1], sa);
      }
    }
    __syncthreads();
    // (2) LDS tile -> global, 16 bytes per lane
    if (!live) {
    } else if constexpr (EPI == EPI_GEGLU) {
      // 32 rows x 32 gated columns: lane (row l/8 + 8u, columns 4*(l%8))
      const int c4 = lane & 7, gc = nw / 2 + 4 * c4;
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int rl = (lane >> 3) + 8 * u, m = m0 + rb + rl;
        const float4 v = *(const float4 *)&tile[rl * LDT + 4 * c4];
        if (m < a.M) {
          float *dst = a.C + (size_t)m * a.ldc + gc;
          if (vec && gc + 4 <= a.n_valid) {
            *(float4 *)dst = v;
          } else {
            const float e[4] = {v.x, v.y, v.z, v.w};
            for (int t = 0; t < 4; t++)
              if (gc + t < a.n_valid) dst[t] = e[t];
          }
        }
      }
    } else if (EPI == EPI_ROPE && nw < a.q_cols) {
      // 32 rows x 64 int8: lane (row l/4 + 16u, bytes 16*(l%4))
      const int8_t *qt = (const int8_t *)tile;
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int rl = (lane >> 2) + 16 * u, m = m0 + rb + rl;
        const v4i v = *(const v4i *)&qt[rl * 64 + 16 * (lane & 3)];
        if (m < a.M) *(v4i *)(a.qq + (size_t)m * a.q_cols + nw + 16 * (lane & 3)) = v;
      }
    } else {
      // 32 rows x 64 values: lane (row l/16 + 4u, columns 4*(l%16))
      const int c4 = lane & 15, col = nw + 4 * c4;
      float4 old[8];
      if constexpr (EPI == EPI_ACCUM || EPI == EPI_ACCUM_MLP) {
#pragma unroll
        for (int u = 0; u < 8; u++) {
          const int m = min(m0 + rb + (lane >> 4) + 4 * u, a.M - 1);
          if (vec && col + 4 <= a.n_valid)
            old[u] = *(const float4 *)(a.C + (size_t)m * a.ldc + col);
          else
            old[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int rl = (lane >> 4) + 4 * u, m = m0 + rb + rl;
        float4 v = *(const float4 *)&tile[rl * LDT + 4 * c4];
        if (m >= a.M) continue;
        if constexpr (EPI == EPI_TILE) {
          int32_t *dst = a.Ci + (size_t)m * a.ldc + col;
          const int e[4] = {__float_as_int(v.x), __float_as_int(v.y), __float_as_int(v.z),
                            __float_as_int(v.w)};
          if (vec && col + 4 <= a.n_valid) {
            *(int4 *)dst = make_int4(e[0], e[1], e[2], e[3]);
          } else {
            for (int t = 0; t < 4; t++)
              if (col + t < a.n_valid) dst[t] = e[t];
          }
        } else {
          float *dst = a.C + (size_t)m * a.ldc + col;
          const bool acc_in = EPI == EPI_ACCUM || EPI == EPI_ACCUM_MLP;
          if (vec && col + 4 <= a.n_valid) {
            if (acc_in)
              v = make_float4(old[u].x + v.x, old[u].y + v.y, old[u].z + v.z, old[u].w + v.w);
            if constexpr (EPI == EPI_ROPE)  // float32 K and V: 256 bytes of a row a quarter-wave, read by the next kernels once
              store_stream_16(dst, v4i{__float_as_int(v.x), __float_as_int(v.y), __float_as_int(v.z), __float_as_int(v.w)});
            else
              *(float4 *)dst = v;
          } else {
            const float e[4] = {v.x, v.y, v.z, v.w};
            for (int t = 0; t < 4; t++)
              if (col + t < a.n_valid) dst[t] = acc_in ? dst[t] + e[t] : e[t];
          }
        }
      }
    }
    __syncthreads();
  }
}

}  // namespace

namespace {

template <int MI, int ST>
void launch_cfg(int epi, const GemmArgs &a, hipStream_t s) {
  using C = Cfg<MI, ST>;
  const int tiles = ((a.M + C::BM - 1) / C::BM) * (a.Np / BN);
  const int per_xcd = (tiles + NXCD - 1) / NXCD;
  const dim3 grid(per_xcd * NXCD), block(256);
  const size_t shm = C::SMEM;
  // up to 72 KB of LDS per workgroup (gfx950 has 160 KB per CU): allow more
  // than the default 64 KB of dynamic LDS, once per kernel instance
  static bool attr_set[8] = {};
  auto launch = [&](auto kern) {
    if (!attr_set[epi]) {
      (void)hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)shm);
      attr_set[epi] = true;
    }
    kern<<<grid, block, shm, s>>>(a);
  };
  switch (epi) {
  case EPI_STORE: launch(gemm_i8_kernel<EPI_STORE, MI, ST>); break;
  case EPI_ACCUM: launch(gemm_i8_kernel<EPI_ACCUM, MI, ST>); break;
  case EPI_TILE: launch(gemm_i8_kernel<EPI_TILE, MI, ST>); break;
  case EPI_GEGLU: launch(gemm_i8_kernel<EPI_GEGLU, MI, ST>); break;
  case EPI_ROPE: launch(gemm_i8_kernel<EPI_ROPE, MI, ST>); break;
  case EPI_ACCUM_MLP: launch(gemm_i8_kernel<EPI_ACCUM_MLP, MI, ST>); break;
  }
}

}  // namespace

void launch_gemm(int epi, const GemmArgs &a, hipStream_t s) {
  if (a.M <= 0) return;
  switch (a.tile_cfg) {
  case 1: launch_cfg<4, 3>(epi, a, s); break;
  case 2: launch_cfg<2, 3>(epi, a, s); break;
  default: launch_cfg<2, 2>(epi, a, s); break;
  }
}

// The int8 MFMA issue rate: every wave of the grid runs `iters` rounds of
// four independent v_mfma_i32_32x32x32_i8 from registers (no memory in the
// loop), then stores a checksum of its accumulators (so that the loop is
// kept).
__global__ __launch_bounds__(256) void mfma_rate_kernel(int iters, int *out) {
  const int t = threadIdx.x;
  const v4i a = {t, 3 * t + 1, 5 * t + 2, 7 * t + 3}, b = {11 * t, 13 * t + 1, 17 * t + 2, 19 * t + 3};
  v16i c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int i = 0; i < iters; i++) {
    c0 = mfma32(a, b, c0);
    c1 = mfma32(b, a, c1);
    c2 = mfma32(a, a, c2);
    c3 = mfma32(b, b, c3);
  }
  int sum = 0;
#pragma unroll
  for (int r = 0; r < 16; r++) sum += c0[r] ^ c1[r] ^ c2[r] ^ c3[r];
  out[(size_t)blockIdx.x * 256 + t] = sum;
}

void launch_mfma_rate(int blocks, int iters, int *out, hipStream_t s) {
  mfma_rate_kernel<<<blocks, 256, 0, s>>>(iters, out);
}

}  // namespace ixh
