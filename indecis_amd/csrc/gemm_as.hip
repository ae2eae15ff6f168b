// gemm_as.hip — the encoder's int8 GEMMs (Wi + GeGLU, Wo and WoMLP +
// residual) with the activation panel resident in LDS and the weights
// streamed straight into registers.
//
// Replaces linalg.MatMul8N (linalg/int8.go:89-155, VNNI tiles
// kernel_vnni_amd64.s:13-256) on the encoder's hot path. Same arithmetic as
// gemm_i8.hip: q*w summed in int32 by v_mfma_i32_32x32x32_i8, the
// reference tile rebuilt as acc + 128*colsum[n], then
// ((f32(tile) - zc[n]) * sb[n]) * sa[m] (+ C) in the reference's order.
//
// Structure (persistent, 2 workgroups of 4 waves per CU):
//  * a unit is (M-block of 32*MB rows, chunk of 256 columns); workgroup r
//    takes a contiguous run of units, so consecutive units mostly share the
//    M-block and its A panel ([32*MB][Kp] int8, 16-byte chunks XOR-swizzled
//    by row & 7) stays in LDS, loaded once with direct-to-LDS loads;
//  * wave w of a unit owns columns 64w..64w+63 of the chunk: no operand is
//    shared between waves except the panel, so the main loop has no
//    barrier. Its B fragments come from the K-blocked weight copy
//    [Kp/32][Np][32] (one MFMA operand = 1 KB contiguous) with buffer
//    loads PF K steps ahead; A fragments are read from LDS one step ahead;
//  * the epilogue of a wave's block (dequantisation, GeGLU or the residual
//    add, stores) runs in slices during the K steps of its next block, so
//    its VALU work and memory traffic issue while the MFMAs of the next
//    block execute. The last block's runs at the end.
// Rows past M and columns past n_valid fall outside the buffer descriptors
// of the stores and loads, which the hardware drops (loads read 0).
#include <algorithm>

#include "ixh_device.h"
#include "ixh_internal.h"

namespace ixh {

namespace gemm_as_impl {

constexpr int NXCD = 8;
constexpr int PF = 4;    // B fragments in flight, in K steps of 32
constexpr int LAG = 2;   // K steps between a residual load and its use
constexpr int CHUNK = 256;  // columns per unit (4 waves x 64)

template <int MB, int KT, int EPI>
__global__ __launch_bounds__(256, 2) void gemm_as_kernel(GemmArgs a, int units, int nchunk) {
  constexpr int BM = 32 * MB, Kp = 32 * KT, CPR = Kp / 16, RS = 16 * MB;
  constexpr int PANEL_INST = BM * Kp / 1024;  // direct-to-LDS instructions per panel
  static_assert(KT % PF == 0 && CPR % 8 == 0, "K must be a multiple of 128");
  extern __shared__ __attribute__((aligned(1024))) int8_t smem[];
  __shared__ float sa_s[2][BM];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 31, fh = lane >> 5;
  // workgroups of one XCD (b % 8) take consecutive runs of units, so an
  // M-block split between two workgroups is read through one L2
  const int G = gridDim.x;
  const int rank = (blockIdx.x % NXCD) * (G / NXCD) + blockIdx.x / NXCD;
  const int u0 = (int)((long long)units * rank / G), u1 = (int)((long long)units * (rank + 1) / G);
  if (u0 >= u1) return;

  // ---- B fragment stream: this wave's column block of each unit, K step
  // by K step, PF steps ahead of the MFMAs (past u1 it reads the next
  // workgroup's columns, in range and unused) ----
  const auto brs = buf_rsrc(a.Bk, (uint32_t)a.Np * Kp);
  const uint32_t bvo = (uint32_t)fr * 32 + 16 * fh;
  int lc = u0 % nchunk, lk = 0;
  auto loadB = [&](v4i *dst) {
    const uint32_t so = __builtin_amdgcn_readfirstlane((uint32_t)lk * a.Np * 32 +
                                                        (uint32_t)((lc * 4 + wave) * 64) * 32);
    dst[0] = __builtin_amdgcn_raw_buffer_load_b128(brs, bvo, so, 0);
    dst[1] = __builtin_amdgcn_raw_buffer_load_b128(brs, bvo + 1024, so, 0);
    if (++lk == KT) {
      lk = 0;
      if (++lc == nchunk) lc = 0;
    }
  };
  v4i bq[PF][2];
#pragma unroll
  for (int s = 0; s < PF; s++) loadB(bq[s]);

  // A fragment of row 32i + fr, K step kt: logical chunk 2kt + fh, stored
  // at chunk (2kt + fh) ^ (fr & 7) = 8(kt/4) + x[kt%4]
  int xo[4];
#pragma unroll
  for (int t = 0; t < 4; t++) xo[t] = fr * Kp + 16 * ((2 * t + fh) ^ (fr & 7));
  v4i fa[2][MB];
  auto loadA = [&](int kt, v4i *dst) {
    const int8_t *p = smem + 128 * (kt >> 2) + xo[kt & 3];
#pragma unroll
    for (int i = 0; i < MB; i++) dst[i] = *(const v4i *)(p + 32 * i * Kp);
  };

  const int ldc = a.ldc;
  v16i acc[MB][2], pacc[MB][2];
  // the pending block (wave-uniform state). Before the first block there is
  // none: its slices run on a descriptor of size 0, so they store nothing.
  // (p_m0 starts past the last row: the phantom block's row maxima are not
  // written either)
  int p_m0 = a.M, p_n = 0, p_par = 0;
  int c1[2];
  float zc[2], sb[2];
  // stores (and EPI_ACCUM's residual loads): C, or Ci for EPI_TILE
  char *const cbase = EPI == EPI_TILE ? (char *)a.Ci : (char *)a.C;
  __amdgpu_buffer_rsrc_t crs = buf_rsrc(cbase, 0);
  uint32_t pvo[2] = {0, 0};
  float old[RS][2];

  // residual loads of slot rs (EPI_ACCUM*)
  auto issue_old = [&](int rs) {
    const int i = rs >> 4, r = rs & 15;
    const uint32_t so = (uint32_t)(32 * i + 8 * (r >> 2) + (r & 3)) * ldc * 4;
#pragma unroll
    for (int jj = 0; jj < 2; jj++)
      old[rs][jj] = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(crs, pvo[jj], so, 0));
  };
  // epilogue of slot rs = (i, r) of the pending block: rows 32i +
  // 8(r/4) + 4fh + r%4, this lane's columns p_n + fr (+32)
  auto process = [&](int rs) {
    const int i = rs >> 4, r = rs & 15;
    const int rw = 32 * i + 8 * (r >> 2) + (r & 3);
    const uint32_t so = (uint32_t)rw * ldc * 4;
    if constexpr (EPI == EPI_TILE) {
#pragma unroll
      for (int jj = 0; jj < 2; jj++)
        __builtin_amdgcn_raw_buffer_store_b32(pacc[i][jj][r] + c1[jj], crs, pvo[jj], so, 0);
    } else {
      const float sa = sa_s[p_par][rw + 4 * fh];
      const float v0 = deq(pacc[i][0][r] + c1[0], zc[0], sb[0], sa);
      const float v1 = deq(pacc[i][1][r] + c1[1], zc[1], sb[1], sa);
      if constexpr (EPI == EPI_GEGLU) {
        // columns p_n..+31: GELU input of gated columns p_n/2 + fr; p_n+32..:
        // their multiplier (Wi rows interleaved by 32; GeluMul
        // vec_simd.go:125-160, FMA form on the multiple-of-16 prefix)
        const int gc = p_n / 2 + fr;
        const float ge = gc < a.n_gelu ? gelu_fma(v0) : gelu_scalar(v0);
        const float gv = ge * v1;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(gv), crs, pvo[0], so, 0);
        if (a.rmax) {
          // max |g| of the row over these 32 gated columns, for the fused
          // residual GEMM that quantises g (quantizeA's max, in parts)
          const float mx = halfwave_max(fabsf(gv));
          const int row = p_m0 + rw + 4 * fh, part = p_n / 64;
          if (fr == 16 && row < a.M && part < a.rmax_ld) a.rmax[(size_t)row * a.rmax_ld + part] = mx;
        }
      } else if constexpr (EPI == EPI_ACCUM || EPI == EPI_ACCUM_MLP) {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(old[rs][0] + v0), crs, pvo[0], so, 0);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(old[rs][1] + v1), crs, pvo[1], so, 0);
      } else {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(v0), crs, pvo[0], so, 0);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(v1), crs, pvo[1], so, 0);
      }
    }
  };
  constexpr bool ACC_IN = EPI == EPI_ACCUM || EPI == EPI_ACCUM_MLP;
  // K step of the slot's residual load / of its epilogue
  auto issue_step = [](int rs) { return rs * (KT - LAG) / RS; };
  auto proc_step = [](int rs) { return ACC_IN ? rs * (KT - LAG) / RS + LAG : rs * KT / RS; };

  int cur_mb = -1, par = 0;
  for (int u = u0; u < u1; u++) {
    const int mb = u / nchunk, c = u - mb * nchunk;
    if (mb != cur_mb) {
      // every wave is done with the panel (its last block's A reads)
      if (cur_mb >= 0) {
        __syncthreads();
        par ^= 1;
      }
      const int m0 = mb * BM;
      for (int t = wave; t < PANEL_INST; t += 4) {
        const int q = 64 * t + lane;
        const int r = q / CPR, ph = q - r * CPR;
        const int row = min(m0 + r, a.M - 1);  // rows past M: never stored
        __builtin_amdgcn_global_load_lds((glb_ptr)(a.A + (size_t)row * a.lda + 16 * (ph ^ (r & 7))),
                                         (lds_ptr)(smem + 1024 * t), 16, 0, 0);
      }
      if (tid < BM) sa_s[par][tid] = a.sa[min(m0 + tid, a.M - 1)];
      wait_vmcnt<0>();
      __syncthreads();
      cur_mb = mb;
    }
    const int n = (c * 4 + wave) * 64;
    loadA(0, fa[0]);
#pragma unroll
    for (int s = 0; s < KT; s++) {
      if constexpr (ACC_IN) {
#pragma unroll
        for (int rs = 0; rs < RS; rs++)
          if (issue_step(rs) == s) issue_old(rs);
      }
      if (s + 1 < KT) loadA(s + 1, fa[(s + 1) & 1]);
      const v4i *f = fa[s & 1];
#pragma unroll
      for (int i = 0; i < MB; i++) {
        acc[i][0] = mfma32(f[i], bq[s % PF][0], s == 0 ? v16i{} : acc[i][0]);
        acc[i][1] = mfma32(f[i], bq[s % PF][1], s == 0 ? v16i{} : acc[i][1]);
      }
      loadB(bq[s % PF]);
#pragma unroll
      for (int rs = 0; rs < RS; rs++)
        if (proc_step(rs) == s) process(rs);
      __builtin_amdgcn_sched_barrier(0);
    }
    // this block becomes the pending one
#pragma unroll
    for (int i = 0; i < MB; i++) {
      pacc[i][0] = acc[i][0];
      pacc[i][1] = acc[i][1];
    }
    p_m0 = mb * BM;
    p_n = n;
    p_par = par;
#pragma unroll
    for (int jj = 0; jj < 2; jj++) {
      const int col = n + 32 * jj + fr;
      c1[jj] = a.c128[col];
      zc[jj] = a.zc[col];
      sb[jj] = a.sb[col];
    }
    // the block's own rows only (at most BM * ldc * 4 bytes, far below 2^31):
    // stores past row M fall outside and are dropped
    crs = buf_rsrc(cbase + (size_t)p_m0 * ldc * 4, (uint32_t)min(a.M - p_m0, BM) * ldc * 4);
    if constexpr (EPI == EPI_GEGLU) {
      const int gc = n / 2 + fr;
      pvo[0] = gc < a.n_valid ? (uint32_t)(4 * fh * ldc + gc) * 4 : 0x80000000u;
    } else {
#pragma unroll
      for (int jj = 0; jj < 2; jj++) {
        const int col = n + 32 * jj + fr;
        pvo[jj] = col < a.n_valid ? (uint32_t)(4 * fh * ldc + col) * 4 : 0x80000000u;
      }
    }
  }
  // the last block, in groups of 8 slots
#pragma unroll
  for (int g = 0; g < RS; g += 8) {
    if constexpr (ACC_IN) {
#pragma unroll
      for (int rs = g; rs < g + 8; rs++) issue_old(rs);
    }
#pragma unroll
    for (int rs = g; rs < g + 8; rs++) process(rs);
  }
}

template <int MB, int KT, int EPI>
void launch_kt(const GemmArgs &a, hipStream_t s) {
  constexpr int BM = 32 * MB;
  const int nchunk = a.Np / CHUNK;
  const int units = ((a.M + BM - 1) / BM) * nchunk;
  int G = std::min(units, 2 * device_cus());
  G = std::max(NXCD, G / NXCD * NXCD);
  const size_t shm = (size_t)BM * 32 * KT;
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute((const void *)gemm_as_kernel<MB, KT, EPI>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    attr = true;
  }
  gemm_as_kernel<MB, KT, EPI><<<G, 256, shm, s>>>(a, units, nchunk);
}

template <int EPI>
bool launch_epi(const GemmArgs &a, hipStream_t s) {
  switch (a.Kp) {
  case 256: launch_kt<2, 8, EPI>(a, s); return true;
  case 512: launch_kt<2, 16, EPI>(a, s); return true;
  case 768: launch_kt<2, 24, EPI>(a, s); return true;
  case 1152: launch_kt<2, 36, EPI>(a, s); return true;
  default: return false;
  }
}

}  // namespace gemm_as_impl

bool gemm_as_supported(const GemmArgs &a) {
  return a.Bk && a.Np % gemm_as_impl::CHUNK == 0 &&
         (a.Kp == 256 || a.Kp == 512 || a.Kp == 768 || a.Kp == 1152);
}

bool launch_gemm_as(int epi, const GemmArgs &a, hipStream_t s) {
  if (a.M <= 0) return true;
  if (!gemm_as_supported(a)) return false;
  switch (epi) {
  case EPI_STORE: return gemm_as_impl::launch_epi<EPI_STORE>(a, s);
  case EPI_ACCUM: return gemm_as_impl::launch_epi<EPI_ACCUM>(a, s);
  case EPI_ACCUM_MLP: return gemm_as_impl::launch_epi<EPI_ACCUM_MLP>(a, s);
  case EPI_TILE: return gemm_as_impl::launch_epi<EPI_TILE>(a, s);
  case EPI_GEGLU: return gemm_as_impl::launch_epi<EPI_GEGLU>(a, s);
  default: return false;
  }
}

}  // namespace ixh
