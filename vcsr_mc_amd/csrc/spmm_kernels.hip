// spmm_kernels.hip -- C += A.B for the VCSR-MC format on gfx950 MFMA.
//
// Work decomposition (atomic-free for all but split panels):
//   one 64-lane wave = one work unit = a run of compacted tiles of one 16-row panel,
//   for one tileK-wide slice of the output columns.  The wave keeps the 16 x tileK
//   accumulator tile in registers across all of its tiles and writes C once.
//
// Per 16 x 32 tile (32 distinct columns of the panel, any segments):
//   * B operand: lane (n = lane % 16, g = lane / 16) loads, for the 8 tile columns
//     k = 8g .. 8g+7, the contiguous VEC = tileK/16 output columns k0 + VEC n .. +VEC-1 of
//     that B row (one 128-bit load per row at tileK = 128, FP16 B); 16 lanes cover a
//     256-byte B row, so every load instruction reads four whole rows.  The VEC values are
//     then transposed in registers: MFMA q (q < VEC) takes the q-th value of each of the 8
//     rows, i.e. output column k0 + VEC n + q.  No LDS round trip for B.
//   * A operand: the tile's nonzeros (row, k, value) are scattered into a 16 x 32 LDS tile
//     that each lane then reads as its 8 contiguous K values (one 128-bit LDS read).
//   * FP16 format: v_mfma_f32_16x16x32_f16, FP32 accumulation.  FP32 format: eight K steps
//     of v_mfma_f32_16x16x4_f32.
//   The K order inside a tile is the same for A and B, so the contraction does not depend
//   on how the instruction maps lanes to K.
//
// Epilogue: lane (n, g) holds rows 4g..4g+3 at output columns k0 + VEC n .. + VEC-1, so each
// row is written as VEC contiguous floats per lane, 16 lanes per row: coalesced.  Rows that
// A does not touch are not written (the reference never touches them either).
#include "../../include/vcsrmc.h"
#include "internal.hpp"

namespace vcsrmc {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kApitch = 40;  // FP16 A tile row pitch in halves (80 B: conflict-free b128 reads)

// Map a linear work-group id to a unit so that each XCD (work-groups are dealt to the 8 XCDs
// round robin) walks a contiguous range of panels: neighbouring panels share B rows in L2.
__device__ __forceinline__ int unit_of_block(int bid, int num_units) {
    const int per = (num_units + 7) >> 3;
    return (bid & 7) * per + (bid >> 3);
}

template <int VEC, typename TB, bool ALIGNED>
__device__ __forceinline__ void load_b_row(const TB* __restrict__ B, int col, long long O, int c0,
                                           _Float16 (&out)[VEC]) {
    if (col < 0) {
#pragma unroll
        for (int q = 0; q < VEC; ++q) out[q] = (_Float16)0.0f;
        return;
    }
    const TB* src = B + (long long)col * O + c0;
    if constexpr (ALIGNED) {
        if (c0 < O) {
            if constexpr (sizeof(TB) == 2) {
                if constexpr (VEC == 1) {
                    out[0] = src[0];
                } else if constexpr (VEC == 8) {
                    const half8 v = *reinterpret_cast<const half8*>(src);
#pragma unroll
                    for (int q = 0; q < 8; ++q) out[q] = v[q];
                } else {
                    typedef _Float16 hv __attribute__((ext_vector_type(VEC)));
                    const hv v = *reinterpret_cast<const hv*>(src);
#pragma unroll
                    for (int q = 0; q < VEC; ++q) out[q] = v[q];
                }
            } else {
                if constexpr (VEC >= 4) {
#pragma unroll
                    for (int h = 0; h < VEC; h += 4) {
                        const floatx4 v = *reinterpret_cast<const floatx4*>(src + h);
#pragma unroll
                        for (int q = 0; q < 4; ++q) out[h + q] = (_Float16)v[q];
                    }
                } else {
#pragma unroll
                    for (int q = 0; q < VEC; ++q) out[q] = (_Float16)src[q];
                }
            }
        } else {
#pragma unroll
            for (int q = 0; q < VEC; ++q) out[q] = (_Float16)0.0f;
        }
    } else {
#pragma unroll
        for (int q = 0; q < VEC; ++q) out[q] = (c0 + q < O) ? (_Float16)src[q] : (_Float16)0.0f;
    }
}

template <int TK, typename TB, bool ALIGNED>
__global__ __launch_bounds__(64) void k_spmm_f16(const int4* __restrict__ units, int num_units,
                                                 const int* __restrict__ chunk_eptr,
                                                 const int* __restrict__ chunk_cols,
                                                 const uint32_t* __restrict__ entries,
                                                 const TB* __restrict__ B, int O, float scale,
                                                 float* __restrict__ C) {
    constexpr int VEC = TK / 16;
    __shared__ __attribute__((aligned(16))) _Float16 As[16 * kApitch];
    const int lane = threadIdx.x, n = lane & 15, g = lane >> 4;
    const int u = unit_of_block(blockIdx.x, num_units);
    if (u >= num_units) return;
    const int4 U = units[u];
    const int k0 = blockIdx.y * TK;
    const int c0 = k0 + VEC * n;
    const long long OL = O;

    floatx4 acc[VEC];
#pragma unroll
    for (int q = 0; q < VEC; ++q) acc[q] = floatx4{0.f, 0.f, 0.f, 0.f};

    _Float16* my_a = &As[n * kApitch + 8 * g];
    for (int c = U.y; c < U.z; ++c) {
        const int4 cl = *reinterpret_cast<const int4*>(chunk_cols + (long long)c * kChunkCols + 8 * g);
        const int4 ch = *reinterpret_cast<const int4*>(chunk_cols + (long long)c * kChunkCols + 8 * g + 4);
        const int cols[8] = {cl.x, cl.y, cl.z, cl.w, ch.x, ch.y, ch.z, ch.w};
        _Float16 R[8][VEC];
#pragma unroll
        for (int i = 0; i < 8; ++i) load_b_row<VEC, TB, ALIGNED>(B, cols[i], OL, c0, R[i]);

        const int eb = chunk_eptr[c], ee = chunk_eptr[c + 1];
        *reinterpret_cast<half8*>(my_a) = half8{0, 0, 0, 0, 0, 0, 0, 0};
        __syncthreads();
        for (int e = eb + lane; e < ee; e += 64) {
            const uint32_t w = entries[e];
            As[((w >> 16) & 15) * kApitch + ((w >> 20) & 31)] =
                __builtin_bit_cast(_Float16, (unsigned short)(w & 0xffffu));
        }
        __syncthreads();
        const half8 a = *reinterpret_cast<const half8*>(my_a);
        __syncthreads();
#pragma unroll
        for (int q = 0; q < VEC; ++q) {
            const half8 b = half8{R[0][q], R[1][q], R[2][q], R[3][q],
                                  R[4][q], R[5][q], R[6][q], R[7][q]};
            acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[q], 0, 0, 0);
        }
    }

    const bool split = (U.w >> 16) & 1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int rl = 4 * g + i;
        if (!((U.w >> rl) & 1)) continue;
        float* crow = C + (long long)(U.x + rl) * OL + c0;
        if (split) {
#pragma unroll
            for (int q = 0; q < VEC; ++q)
                if (c0 + q < O) atomicAdd(crow + q, acc[q][i] * scale);
        } else {
            if constexpr (ALIGNED && VEC >= 4) {
                if (c0 < O) {
#pragma unroll
                    for (int h = 0; h < VEC; h += 4) {
                        floatx4 v = *reinterpret_cast<floatx4*>(crow + h);
#pragma unroll
                        for (int q = 0; q < 4; ++q) v[q] += acc[h + q][i] * scale;
                        *reinterpret_cast<floatx4*>(crow + h) = v;
                    }
                }
            } else {
#pragma unroll
                for (int q = 0; q < VEC; ++q)
                    if (c0 + q < O) crow[q] += acc[q][i] * scale;
            }
        }
    }
}

template <int VEC, bool ALIGNED>
__device__ __forceinline__ void load_b_row_f32(const float* __restrict__ B, int col, long long O,
                                               int c0, float (&out)[VEC]) {
    if (col < 0) {
#pragma unroll
        for (int q = 0; q < VEC; ++q) out[q] = 0.0f;
        return;
    }
    const float* src = B + (long long)col * O + c0;
    if constexpr (ALIGNED && VEC >= 4) {
        if (c0 < O) {
#pragma unroll
            for (int h = 0; h < VEC; h += 4) {
                const floatx4 v = *reinterpret_cast<const floatx4*>(src + h);
#pragma unroll
                for (int q = 0; q < 4; ++q) out[h + q] = v[q];
            }
        } else {
#pragma unroll
            for (int q = 0; q < VEC; ++q) out[q] = 0.0f;
        }
    } else {
#pragma unroll
        for (int q = 0; q < VEC; ++q) out[q] = (c0 + q < O) ? src[q] : 0.0f;
    }
}

// FP32 format: A tile stored K-step-major so a lane's 8 K values (k = 4s + g, s = 0..7) are
// contiguous: At[(k & 3) * 128 + row * 8 + (k >> 2)].
template <int TK, bool ALIGNED>
__global__ __launch_bounds__(64) void k_spmm_f32(const int4* __restrict__ units, int num_units,
                                                 const int* __restrict__ chunk_eptr,
                                                 const int* __restrict__ chunk_cols,
                                                 const uint32_t* __restrict__ entries,
                                                 const float* __restrict__ evals,
                                                 const float* __restrict__ B, int O,
                                                 float* __restrict__ C) {
    constexpr int VEC = TK / 16;
    __shared__ __attribute__((aligned(16))) float At[4 * 16 * 8];
    const int lane = threadIdx.x, n = lane & 15, g = lane >> 4;
    const int u = unit_of_block(blockIdx.x, num_units);
    if (u >= num_units) return;
    const int4 U = units[u];
    const int k0 = blockIdx.y * TK;
    const int c0 = k0 + VEC * n;
    const long long OL = O;

    floatx4 acc[VEC];
#pragma unroll
    for (int q = 0; q < VEC; ++q) acc[q] = floatx4{0.f, 0.f, 0.f, 0.f};

    float* my_a = &At[g * 128 + n * 8];
    for (int c = U.y; c < U.z; ++c) {
        const int* cc = chunk_cols + (long long)c * kChunkCols;
        int cols[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) cols[s] = cc[4 * s + g];
        float R[8][VEC];
#pragma unroll
        for (int s = 0; s < 8; ++s) load_b_row_f32<VEC, ALIGNED>(B, cols[s], OL, c0, R[s]);

        const int eb = chunk_eptr[c], ee = chunk_eptr[c + 1];
        *reinterpret_cast<floatx4*>(my_a) = floatx4{0.f, 0.f, 0.f, 0.f};
        *reinterpret_cast<floatx4*>(my_a + 4) = floatx4{0.f, 0.f, 0.f, 0.f};
        __syncthreads();
        for (int e = eb + lane; e < ee; e += 64) {
            const uint32_t w = entries[e];
            const int r = w & 15, k = (w >> 4) & 31;
            At[(k & 3) * 128 + r * 8 + (k >> 2)] = evals[e];
        }
        __syncthreads();
        const floatx4 a_lo = *reinterpret_cast<const floatx4*>(my_a);
        const floatx4 a_hi = *reinterpret_cast<const floatx4*>(my_a + 4);
        __syncthreads();
        const float a[8] = {a_lo[0], a_lo[1], a_lo[2], a_lo[3], a_hi[0], a_hi[1], a_hi[2], a_hi[3]};
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            if (__ballot(cols[s] >= 0) == 0) break;  // padding columns sit at the end of a tile
#pragma unroll
            for (int q = 0; q < VEC; ++q)
                acc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], R[s][q], acc[q], 0, 0, 0);
        }
    }

    const bool split = (U.w >> 16) & 1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int rl = 4 * g + i;
        if (!((U.w >> rl) & 1)) continue;
        float* crow = C + (long long)(U.x + rl) * OL + c0;
        if (split) {
#pragma unroll
            for (int q = 0; q < VEC; ++q)
                if (c0 + q < O) atomicAdd(crow + q, acc[q][i]);
        } else {
            if constexpr (ALIGNED && VEC >= 4) {
                if (c0 < O) {
#pragma unroll
                    for (int h = 0; h < VEC; h += 4) {
                        floatx4 v = *reinterpret_cast<floatx4*>(crow + h);
#pragma unroll
                        for (int q = 0; q < 4; ++q) v[q] += acc[h + q][i];
                        *reinterpret_cast<floatx4*>(crow + h) = v;
                    }
                }
            } else {
#pragma unroll
                for (int q = 0; q < VEC; ++q)
                    if (c0 + q < O) crow[q] += acc[q][i];
            }
        }
    }
}

template <int TK>
static void launch_tk(const DeviceFormat& F, const void* dB, bool b_f16, int O, float* dC,
                      hipStream_t st) {
    constexpr int VEC = TK / 16;
    // Vector loads of B and the float4 epilogue need O % VEC == 0 and 16-byte aligned bases.
    const bool aligned = (O % VEC) == 0 && ((uintptr_t)dB % 16) == 0 && ((uintptr_t)dC % 16) == 0;
    const dim3 grid((unsigned)(8 * ((F.num_units + 7) / 8)), (unsigned)((O + TK - 1) / TK));
    const dim3 block(64);
    if (F.fp32) {
        const float* B = static_cast<const float*>(dB);
        if (aligned)
            hipLaunchKernelGGL((k_spmm_f32<TK, true>), grid, block, 0, st, F.units.p, F.num_units,
                               F.chunk_eptr.p, F.chunk_cols.p, F.entries.p, F.evals.p, B, O, dC);
        else
            hipLaunchKernelGGL((k_spmm_f32<TK, false>), grid, block, 0, st, F.units.p, F.num_units,
                               F.chunk_eptr.p, F.chunk_cols.p, F.entries.p, F.evals.p, B, O, dC);
    } else if (b_f16) {
        const _Float16* B = static_cast<const _Float16*>(dB);
        if (aligned)
            hipLaunchKernelGGL((k_spmm_f16<TK, _Float16, true>), grid, block, 0, st, F.units.p,
                               F.num_units, F.chunk_eptr.p, F.chunk_cols.p, F.entries.p, B, O,
                               F.scale, dC);
        else
            hipLaunchKernelGGL((k_spmm_f16<TK, _Float16, false>), grid, block, 0, st, F.units.p,
                               F.num_units, F.chunk_eptr.p, F.chunk_cols.p, F.entries.p, B, O,
                               F.scale, dC);
    } else {
        const float* B = static_cast<const float*>(dB);
        if (aligned)
            hipLaunchKernelGGL((k_spmm_f16<TK, float, true>), grid, block, 0, st, F.units.p,
                               F.num_units, F.chunk_eptr.p, F.chunk_cols.p, F.entries.p, B, O,
                               F.scale, dC);
        else
            hipLaunchKernelGGL((k_spmm_f16<TK, float, false>), grid, block, 0, st, F.units.p,
                               F.num_units, F.chunk_eptr.p, F.chunk_cols.p, F.entries.p, B, O,
                               F.scale, dC);
    }
    VCSRMC_HIP(hipGetLastError());
}

void spmm_launch(const DeviceFormat& F, const void* dB, bool b_f16, int O, int tileK, float* dC,
                 hipStream_t st) {
    if (tileK != 16 && tileK != 32 && tileK != 64 && tileK != 128)
        throw Error(VCSRMC_ERR_TILEK, "vcsr_mc supports tileK in {16, 32, 64, 128}");
    if (!F.ready) throw Error(VCSRMC_ERR_STATE, "no format in this handle");
    if (O < 0) throw Error(VCSRMC_ERR_ARG, "O must be >= 0");
    if (F.fp32 && b_f16) throw Error(VCSRMC_ERR_ARG, "an FP32 format takes an FP32 B");
    if (F.num_units == 0 || O == 0) return;
    if (!dB || !dC) throw Error(VCSRMC_ERR_ARG, "null B or C");
    switch (tileK) {
        case 16: launch_tk<16>(F, dB, b_f16, O, dC, st); break;
        case 32: launch_tk<32>(F, dB, b_f16, O, dC, st); break;
        case 64: launch_tk<64>(F, dB, b_f16, O, dC, st); break;
        default: launch_tk<128>(F, dB, b_f16, O, dC, st); break;
    }
}

}  // namespace vcsrmc
