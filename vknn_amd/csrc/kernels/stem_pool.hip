// First layer + 3x3 stride-2 max pool in one kernel (the ResNet stem: 7x7/s2 conv, ReLU, 3x3/s2
// pad-1 max pool). The reference runs them as two ops (src/backend/vulkan/ops/conv.cpp and
// ops/pool.cpp, shaders/maxpool.comp), so the 112x112x64 conv output makes a round trip through
// memory; here it lives only in LDS.
//
// One workgroup (8 waves) owns PR pooled rows of one image. It computes the 2*PR+1 conv output
// rows those rows pool over (the first one shared with the previous workgroup, which computes it
// too) exactly as conv_stem_kernel does — weights and the input band copied into LDS by
// buffer-load-to-LDS, four taps per 16-deep MFMA K step — then writes the conv tile (bias,
// activation, RNE fp16) into LDS over the band, and pools it: each output is the fp16 max of the
// in-image taps of its 3x3 window, the same packed max the max-pool kernel uses, so the result is
// bit-identical to the two unfused kernels.
#include "conv_kernels.h"

namespace vkhip {

    typedef _Float16 half2v __attribute__((ext_vector_type(2)));

    template <int K, int FN, int WN>
    __global__ __launch_bounds__(64 * WN) void stem_pool_kernel(GemmArgs a, uint2 *py, int POH, int POW, int PR, int NBI) {
        constexpr int FM = 2, NW = WN;
        constexpr int BN = 32 * FN * WN;
        constexpr int LDS = stem_pool_lds(FN, WN);
        constexpr int MF     = FM;
        constexpr int KT     = (K * K + 3) / 4;
        constexpr int KH2    = K / 2;
        constexpr int NA     = KT * MF;        // 1 KB weight chunks
        constexpr int BOFF   = NA * 1024 + 32; // band start (32 zero guard bytes before it)
        __shared__ __attribute__((aligned(16))) unsigned char sm[LDS];
        const int SPARE = LDS - 1024;

        const int tid  = threadIdx.x;
        const int lane = tid & 63;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int wn0  = wave * 32 * FN;
        const int groups = (POH + PR - 1) / PR;
        const int n      = blockIdx.x / groups;
        const int py0    = (blockIdx.x - n * groups) * PR;
        const int oyA    = 2 * py0 - 1;       // first conv row of the tile (-1 for the first group)
        const int R      = 2 * PR + 1;

        const int W = a.W, H = a.H, OW = a.OW, S = a.SH;
        const int OH   = a.OHW / OW;
        const int RS   = W + K - 1;           // band row stride in pixels
        const int VRB  = S * (R - 1) + K;     // band rows
        const int iyB  = S * oyA - KH2;       // input row of band row 0
        const int NC   = NA + NBI;
        const int NCW  = (NC + NW - 1) / NW;

        const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void *) a.x, (short) 0, (int) a.x_bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc((void *) a.w, (short) 0, NA * 1024, 0x00020000);
        constexpr unsigned kInvalid = 0x80000000u;
        if (tid < 2) *reinterpret_cast<u32x4 *>(&sm[NA * 1024 + tid * 16]) = u32x4 {0u, 0u, 0u, 0u};

        // copies: chunk c = r*NW + wave; chunks < NA are weights, then NBI band chunks (pixel pairs,
        // row-major over band rows), the rest copy zeros into the spare KB
        for (int r = 0; r < NCW; ++r) {
            const int c = r * NW + wave;
            if (c < NA) {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (__attribute__((address_space(3))) void *) (sm + c * 1024), 16,
                                                         (unsigned) (c * 1024 + lane * 16), 0, 0, 0);
            } else {
                const int  k    = (c - NA) * 64 + lane;
                const int  vrow = k / (RS >> 1);
                const int  pc   = k - vrow * (RS >> 1);
                const int  iy   = iyB + vrow;
                const bool ok   = c < NC && 2 * pc < W && iy >= 0 && iy < H && vrow < VRB;
                const unsigned vo = ok ? (unsigned) ((n * a.HW + iy * W + 2 * pc) * 8) : kInvalid;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (__attribute__((address_space(3))) void *) (c < NC ? sm + BOFF + (c - NA) * 1024 : sm + SPARE),
                                                         16, vo, 0, 0, 0);
            }
        }

        // per lane: band position of each fragment column's centre tap, and the two tap offsets of
        // every K step
        const int g = lane >> 5;
        int       qb[FN];
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int q = wn0 + 32 * j + (lane & 31); // tile column: conv row oyA + q / OW, column q % OW
            int       p = KH2 * RS + KH2;             // any interior position for columns outside the tile
            if (q < R * OW) {
                const int r = q / OW, ox = q - r * OW;
                p           = (S * r + KH2) * RS + S * ox;
            }
            qb[j] = BOFF + p * 8;
        }
        int toff[KT][2];
#pragma unroll
        for (int s = 0; s < KT; ++s)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int t = 4 * s + 2 * g + h;
                toff[s][h]  = t < K * K ? ((t / K - KH2) * RS + (t % K - KH2)) * 8 : 0;
            }

        float16v acc[FM][FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

        __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
        __syncthreads();
        const unsigned char *Ab = sm + lane * 16;
        half8 fa[2][FM], fb[2][FN];
        auto rd = [&](int s, int d) __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const u32x2 lo = *reinterpret_cast<const u32x2 *>(sm + qb[j] + toff[s][0]);
                const u32x2 hi = *reinterpret_cast<const u32x2 *>(sm + qb[j] + toff[s][1]);
                fb[d][j] = __builtin_bit_cast(half8, u32x4_make(lo.x, lo.y, hi.x, hi.y));
            }
#pragma unroll
            for (int i = 0; i < FM; ++i) fa[d][i] = *reinterpret_cast<const half8 *>(Ab + (s * MF + i) * 1024);
        };
        rd(0, 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < KT; ++s) {
            if (s + 1 < KT) rd(s + 1, (s + 1) & 1);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[s & 1][i], fb[s & 1][j], acc[i][j], 0, 0, 0);
            if (s + 1 < KT) StepSchedule<0, FM * FN, FM + 2 * FN, 4 * FN>::apply();
            __builtin_amdgcn_sched_barrier(0);
        }

        // conv tile -> LDS (over the band): [channel block][tile column], bias + activation, RNE fp16
        __syncthreads();
        uint2    *tile = reinterpret_cast<uint2 *>(sm);
        const int lk   = lane >> 5;
        auto finish = [&](auto act_c) __attribute__((always_inline)) {
            constexpr int ACT = decltype(act_c)::value;
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int qq = 0; qq < 4; ++qq) {
                    const int     oc = i * 32 + qq * 8 + lk * 4;
                    const float4v bv = *reinterpret_cast<const float4v *>(a.bias + oc);
#pragma unroll
                    for (int j = 0; j < FN; ++j) {
                        const int q = wn0 + 32 * j + (lane & 31);
                        if (q >= R * OW) continue;
                        float4v v = {acc[i][j][qq * 4 + 0], acc[i][j][qq * 4 + 1], acc[i][j][qq * 4 + 2], acc[i][j][qq * 4 + 3]};
                        v += bv;
                        v.x = apply_act(v.x, ACT, a.lo, a.hi);
                        v.y = apply_act(v.y, ACT, a.lo, a.hi);
                        v.z = apply_act(v.z, ACT, a.lo, a.hi);
                        v.w = apply_act(v.w, ACT, a.lo, a.hi);
                        if (oc + 0 >= a.Cout) v.x = 0.f;
                        if (oc + 1 >= a.Cout) v.y = 0.f;
                        if (oc + 2 >= a.Cout) v.z = 0.f;
                        if (oc + 3 >= a.Cout) v.w = 0.f;
                        tile[(oc >> 2) * BN + q] = h4_as_u2(f4_to_h4(v));
                    }
                }
        };
        switch (a.act) {
            case VKHIP_ACT_RELU: finish(std::integral_constant<int, VKHIP_ACT_RELU> {}); break;
            case VKHIP_ACT_RELU6: finish(std::integral_constant<int, VKHIP_ACT_RELU6> {}); break;
            case VKHIP_ACT_CLIP: finish(std::integral_constant<int, VKHIP_ACT_CLIP> {}); break;
            case VKHIP_ACT_HARDSWISH: finish(std::integral_constant<int, VKHIP_ACT_HARDSWISH> {}); break;
            case VKHIP_ACT_SILU: finish(std::integral_constant<int, VKHIP_ACT_SILU> {}); break;
            default: finish(std::integral_constant<int, VKHIP_ACT_NONE> {}); break;
        }
        __syncthreads();

        // 3x3 stride-2 pad-1 max pool of the tile: output (py, px) takes conv rows 2py-1 .. 2py+1
        // (tile rows 2(py-py0) .. +2) and columns 2px-1 .. 2px+1 that lie inside the conv output
        const int prv   = min(PR, POH - py0);
        const int items = a.Coutb * prv * POW;
        const half2v ninf = __builtin_bit_cast(half2v, 0xFC00FC00u);
        for (int it = tid; it < items; it += 64 * NW) {
            const int cb  = it / (prv * POW);
            const int rem = it - cb * prv * POW;
            const int pyl = rem / POW, px = rem - pyl * POW;
            half2v    m0 = ninf, m1 = ninf;
#pragma unroll
            for (int dy = 0; dy < 3; ++dy) {
                const int oy = oyA + 2 * pyl + dy;
                if (oy < 0 || oy >= OH) continue;
#pragma unroll
                for (int dx = 0; dx < 3; ++dx) {
                    const int ox = 2 * px - 1 + dx;
                    if (ox < 0 || ox >= OW) continue;
                    const uint2 v = tile[cb * BN + (2 * pyl + dy) * OW + ox];
                    m0 = __builtin_elementwise_max(m0, __builtin_bit_cast(half2v, v.x));
                    m1 = __builtin_elementwise_max(m1, __builtin_bit_cast(half2v, v.y));
                }
            }
            py[(((long long) n * a.Coutb + cb) * POH + py0 + pyl) * POW + px] = uint2 {__builtin_bit_cast(unsigned, m0), __builtin_bit_cast(unsigned, m1)};
        }
    }

    StemPoolFn stem_pool_kernel_for(int K, int cfg) {
        if (K == 7) return cfg == 0 ? stem_pool_kernel<7, kSP0FN, kSP0WN> : stem_pool_kernel<7, kSP1FN, kSP1WN>;
        if (K == 3) return cfg == 0 ? stem_pool_kernel<3, kSP0FN, kSP0WN> : stem_pool_kernel<3, kSP1FN, kSP1WN>;
        return nullptr;
    }

} // namespace vkhip
