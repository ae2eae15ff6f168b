// gemm_ws.hip — the encoder's int8 GEMMs with warp-specialised waves:
// MFMA waves that only compute, epilogue waves that only dequantise, apply
// GeGLU or the residual add, and store.
//
// Replaces linalg.MatMul8N (linalg/int8.go:89-155, VNNI tiles
// kernel_vnni_amd64.s:13-256) for Wi + GeGLU (GeluMul, vec_simd.go:125-160)
// and the residual GEMMs Wo, WoMLP (infer.go:403,423). Same arithmetic as
// gemm_i8.hip: q*w summed in int32 by v_mfma_i32_32x32x32_i8, the
// reference tile rebuilt as acc + 128*colsum[n], then
// ((f32(tile) - zc[n]) * sb[n]) * sa[m] (+ C) in the reference's order.
//
// One persistent workgroup of 8 waves per CU; waves 0-3 compute, waves 4-7
// finish (wave w and w+4 share a SIMD and a column block):
//  * a unit is (M-block of 64 rows, chunk of 256 columns); a workgroup
//    takes a contiguous run of units, the M-block's A panel ([64][Kp] int8,
//    16-byte chunks XOR-swizzled by row & 7) stays in LDS while the run
//    stays in the M-block;
//  * MFMA wave w owns columns 64w..64w+63 of the unit. Its B fragments
//    stream from the K-blocked weights [Kp/32][Np][32] (1 KB contiguous per
//    MFMA operand) PF K steps ahead, its A fragments come from the panel one
//    step ahead. No other loads: the in-order vmcnt never waits on HBM;
//  * after a block's K loop the MFMA wave writes its 64x64 int32 sums to
//    LDS (two workgroup barriers: the buffer is free, the buffer is full)
//    and goes on with the next block, while epilogue wave w+4 reads them
//    into registers and finishes them in the shadow of the next K loop:
//    row-major, 16 bytes per lane, residual rows loaded all at once.
// Rows past M and columns past n_valid fall outside the buffer descriptors
// of the stores and loads, which the hardware drops (loads read 0).
// The 16-byte stores take their whole offset in the VGPR (SGPR offset 0):
// the compiler adds wait states between such a store and a VALU write of
// its data registers only when the SGPR offset is the constant 0, and with
// an SGPR there, a register reused right after the store was seen to change
// the stored dword on gfx950.
#include <algorithm>

#include "ixh_device.h"
#include "ixh_internal.h"

namespace ixh {

namespace gemm_ws_impl {

constexpr int NXCD = 8;
constexpr int PF = 4;       // B fragments in flight, in K steps of 32
constexpr int CHUNK = 256;  // columns per unit (4 MFMA waves x 64)
constexpr int BM = 64;      // rows per M-block
constexpr int HLD = 68;     // int32 per row of a handover tile (64 + 4)
constexpr int HAND_BYTES = 4 * BM * HLD * 4;

// Workgroup barrier for LDS hand-offs: this wave's LDS accesses complete
// (lgkmcnt 0), then s_barrier. Unlike __syncthreads it does not wait for the
// wave's global loads, so the MFMA waves keep their weight stream in flight.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // vmcnt 63, expcnt 7, lgkmcnt 0
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int KT, int EPI>
__global__ __launch_bounds__(512) void gemm_ws_kernel(GemmArgs a, int units, int nchunk) {
  constexpr int Kp = 32 * KT, CPR = Kp / 16, PANEL = BM * Kp;
  static_assert(KT % PF == 0 && CPR % 8 == 0, "K must be a multiple of 128");
  constexpr bool ACC_IN = EPI == EPI_ACCUM || EPI == EPI_ACCUM_MLP;
  extern __shared__ __attribute__((aligned(1024))) int8_t smem[];
  int32_t *const hand_all = (int32_t *)(smem + PANEL);
  __shared__ float sa_s[2][BM];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool mfma_wave = wave < 4;
  const int cw = wave & 3;  // column block of the unit (both roles)
  int32_t *const hand = hand_all + cw * BM * HLD;
  const int G = gridDim.x;
  const int rank = (blockIdx.x % NXCD) * (G / NXCD) + blockIdx.x / NXCD;
  const int u0 = (int)((long long)units * rank / G), u1 = (int)((long long)units * (rank + 1) / G);
  if (u0 >= u1) return;
  const int ldc = a.ldc;

  // ---- MFMA-wave state ----
  const int fr = lane & 31, fh = lane >> 5;
  const auto brs = buf_rsrc(a.Bk, (uint32_t)a.Np * Kp);
  const uint32_t bvo = (uint32_t)fr * 32 + 16 * fh;
  int lc = u0 % nchunk, lk = 0;
  auto loadB = [&](v4i *dst) {
    const uint32_t so = __builtin_amdgcn_readfirstlane((uint32_t)lk * a.Np * 32 +
                                                        (uint32_t)((lc * 4 + cw) * 64) * 32);
    dst[0] = __builtin_amdgcn_raw_buffer_load_b128(brs, bvo, so, 0);
    dst[1] = __builtin_amdgcn_raw_buffer_load_b128(brs, bvo + 1024, so, 0);
    if (++lk == KT) {
      lk = 0;
      if (++lc == nchunk) lc = 0;
    }
  };
  v4i bq[PF][2];
  int xo[4];
#pragma unroll
  for (int t = 0; t < 4; t++) xo[t] = fr * Kp + 16 * ((2 * t + fh) ^ (fr & 7));

  // ---- epilogue-wave state: the block taken from the handover tile ----
  // lane: column group cg (4 columns; GEGLU: 4 gated columns), rows
  // rg + RSTEP*t
  constexpr int NCG = EPI == EPI_GEGLU ? 8 : 16;  // column groups per row
  constexpr int RSTEP = 64 / NCG;                 // rows per instruction
  constexpr int NT = BM / RSTEP;                  // row steps per lane
  const int cg = lane % NCG, rg = lane / NCG;
  v4i pv[NT][EPI == EPI_GEGLU ? 2 : 1];  // the sums (GEGLU: input, gate)
  float4 old[NT];
  int p_m0 = 0, p_n = 0, p_par = 0;
  __amdgpu_buffer_rsrc_t crs = buf_rsrc(a.C, 0);
  char *const cbase = EPI == EPI_TILE ? (char *)a.Ci : (char *)a.C;
  uint32_t pvo = 0;

  // take the handover tile into registers and start its residual loads
  auto take = [&](int m0, int n, int tpar) {
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const int32_t *row = hand + (rg + RSTEP * t) * HLD;
      pv[t][0] = *(const v4i *)(row + 4 * cg);
      if constexpr (EPI == EPI_GEGLU) pv[t][1] = *(const v4i *)(row + 32 + 4 * cg);
    }
    p_m0 = m0;
    p_n = n;
    p_par = tpar;
    // the block's own rows only (at most BM * ldc * 4 bytes): rows past M
    // fall outside and are dropped
    crs = buf_rsrc(cbase + (size_t)m0 * ldc * 4, (uint32_t)min(a.M - m0, BM) * ldc * 4);
    const int col = EPI == EPI_GEGLU ? n / 2 + 4 * cg : n + 4 * cg;
    pvo = col < a.n_valid ? (uint32_t)(rg * ldc + col) * 4 : 0x80000000u;
    if constexpr (ACC_IN) {
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const v4i o = __builtin_amdgcn_raw_buffer_load_b128(crs, pvo + (uint32_t)(RSTEP * t) * ldc * 4, 0, 0);
        old[t] = make_float4(__int_as_float(o[0]), __int_as_float(o[1]), __int_as_float(o[2]),
                             __int_as_float(o[3]));
      }
    }
  };
  // finish the taken block
  auto finish = [&]() {
    const int c0 = p_n + 4 * cg;
    int c1[2][4];
    float zc[2][4], sb[2][4];
#pragma unroll
    for (int h = 0; h < (EPI == EPI_GEGLU ? 2 : 1); h++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int col = c0 + 32 * h + e;
        c1[h][e] = a.c128[col];
        zc[h][e] = a.zc[col];
        sb[h][e] = a.sb[col];
      }
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const uint32_t vo = pvo + (uint32_t)(RSTEP * t) * ldc * 4;
      const float sa = sa_s[p_par][rg + RSTEP * t];
      float o[4];
      if constexpr (EPI == EPI_TILE) {
        v4i r;
#pragma unroll
        for (int e = 0; e < 4; e++) r[e] = pv[t][0][e] + c1[0][e];
        __builtin_amdgcn_raw_buffer_store_b128(r, crs, vo, 0, 0);
        continue;
      } else {
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float v = deq(pv[t][0][e] + c1[0][e], zc[0][e], sb[0][e], sa);
          if constexpr (EPI == EPI_GEGLU) {
            // gated column p_n/2 + 4cg + e: GELU of column p_n + 4cg + e
            // times column p_n + 32 + 4cg + e (Wi rows interleaved by 32)
            const float vb = deq(pv[t][1][e] + c1[1][e], zc[1][e], sb[1][e], sa);
            const int gc = p_n / 2 + 4 * cg + e;
            o[e] = (gc < a.n_gelu ? gelu_fma(v) : gelu_scalar(v)) * vb;
          } else {
            o[e] = v;
          }
        }
        if constexpr (ACC_IN) {
          o[0] = old[t].x + o[0];
          o[1] = old[t].y + o[1];
          o[2] = old[t].z + o[2];
          o[3] = old[t].w + o[3];
        }
        const v4i r = {__float_as_int(o[0]), __float_as_int(o[1]), __float_as_int(o[2]),
                       __float_as_int(o[3])};
        __builtin_amdgcn_raw_buffer_store_b128(r, crs, vo, 0, 0);
      }
    }
  };

  // The two roles run separate loops (their live registers do not add up);
  // each unit both pass the same barriers: P (a new panel is in LDS), X (the
  // handover tile is free), Y (it is full).
  auto load_panel = [&](int mb, int par) {
    const int m0 = mb * BM;
    for (int t = wave; t < PANEL / 1024; t += 8) {
      const int q = 64 * t + lane;
      const int r = q / CPR, ph = q - r * CPR;
      const int row = min(m0 + r, a.M - 1);  // rows past M: never stored
      __builtin_amdgcn_global_load_lds((glb_ptr)(a.A + (size_t)row * a.lda + 16 * (ph ^ (r & 7))),
                                       (lds_ptr)(smem + 1024 * t), 16, 0, 0);
    }
    if (tid < BM) sa_s[par][tid] = a.sa[min(m0 + tid, a.M - 1)];
    wait_vmcnt<0>();
    lds_barrier();  // P
  };
  int cur_mb = -1, par = 0;
  if (mfma_wave) {
#pragma unroll
    for (int s = 0; s < PF; s++) loadB(bq[s]);
    for (int u = u0; u < u1; u++) {
      const int mb = u / nchunk;
      if (mb != cur_mb) {
        // past barrier Y of the previous unit: no wave reads the old panel
        if (cur_mb >= 0) par ^= 1;
        load_panel(mb, par);
        cur_mb = mb;
      }
      v16i acc[2][2];
      v4i fa[2][2];
      auto loadA = [&](int kt, v4i *dst) {
        const int8_t *p = smem + 128 * (kt >> 2) + xo[kt & 3];
        dst[0] = *(const v4i *)p;
        dst[1] = *(const v4i *)(p + 32 * Kp);
      };
      loadA(0, fa[0]);
#pragma unroll
      for (int s = 0; s < KT; s++) {
        if (s + 1 < KT) loadA(s + 1, fa[(s + 1) & 1]);
        const v4i *f = fa[s & 1];
#pragma unroll
        for (int i = 0; i < 2; i++) {
          acc[i][0] = mfma32(f[i], bq[s % PF][0], s == 0 ? v16i{} : acc[i][0]);
          acc[i][1] = mfma32(f[i], bq[s % PF][1], s == 0 ? v16i{} : acc[i][1]);
        }
        loadB(bq[s % PF]);
        __builtin_amdgcn_sched_barrier(0);
      }
      lds_barrier();  // X
      // sums -> handover tile, row-major: element (32i + acc_row(r), 32jj + fr)
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int jj = 0; jj < 2; jj++)
#pragma unroll
          for (int r = 0; r < 16; r++)
            hand[(32 * i + acc_row(r, lane)) * HLD + 32 * jj + fr] = acc[i][jj][r];
      lds_barrier();  // Y
    }
  } else {
    bool have = false;
    for (int u = u0; u < u1; u++) {
      const int mb = u / nchunk, c = u - mb * nchunk;
      if (mb != cur_mb) {
        if (cur_mb >= 0) par ^= 1;
        load_panel(mb, par);
        cur_mb = mb;
      }
      if (have) finish();
      lds_barrier();  // X
      lds_barrier();  // Y
      take(mb * BM, (c * 4 + cw) * 64, par);
      have = true;
    }
    finish();
  }
}

template <int KT, int EPI>
void launch_kt(const GemmArgs &a, hipStream_t s) {
  const int nchunk = a.Np / CHUNK;
  const int units = ((a.M + BM - 1) / BM) * nchunk;
  int G = std::min(units, device_cus());
  G = std::max(NXCD, G / NXCD * NXCD);
  const size_t shm = (size_t)BM * 32 * KT + HAND_BYTES;
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute((const void *)gemm_ws_kernel<KT, EPI>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    attr = true;
  }
  gemm_ws_kernel<KT, EPI><<<G, 512, shm, s>>>(a, units, nchunk);
}

template <int EPI>
bool launch_epi(const GemmArgs &a, hipStream_t s) {
  switch (a.Kp) {
  case 256: launch_kt<8, EPI>(a, s); return true;
  case 512: launch_kt<16, EPI>(a, s); return true;
  case 768: launch_kt<24, EPI>(a, s); return true;
  case 1152: launch_kt<36, EPI>(a, s); return true;
  default: return false;
  }
}

}  // namespace gemm_ws_impl

bool launch_gemm_ws(int epi, const GemmArgs &a, hipStream_t s) {
  if (a.M <= 0) return true;
  if (!gemm_as_supported(a)) return false;
  switch (epi) {
  case EPI_STORE: return gemm_ws_impl::launch_epi<EPI_STORE>(a, s);
  case EPI_ACCUM: return gemm_ws_impl::launch_epi<EPI_ACCUM>(a, s);
  case EPI_ACCUM_MLP: return gemm_ws_impl::launch_epi<EPI_ACCUM_MLP>(a, s);
  case EPI_TILE: return gemm_ws_impl::launch_epi<EPI_TILE>(a, s);
  case EPI_GEGLU: return gemm_ws_impl::launch_epi<EPI_GEGLU>(a, s);
  default: return false;
  }
}

}  // namespace ixh
