// A ResNet-style stem and its max pool in one kernel: a 7x7 stride-2 pad-3 conv over at most 4
// input channels to at most 64 channels, then the 3x3 stride-2 pad-1 max pool over its output
// (ResNet-50: 3 -> 64 at 224x224, pooled to 56x56). Run as two launches, the conv output (103 MB at
// b64) is written and read back; here it stays in LDS:
//   * one persistent workgroup per CU slot walks items of 2 pooled rows x up to 28 pooled columns
//     (the pooled width split evenly), XCD-contiguous item ranges;
//   * the item's input band (15 rows of the input's 4-channel slot) arrives in LDS by
//     buffer-load-to-LDS; the next item's band is issued as soon as this item's conv has read it,
//     so it streams in under the pool phase;
//   * the conv computes the 5 rows x (2 pw + 1) columns its pool windows cover (the row shared by
//     two items is computed by both) on 16x16x32 MFMA with the weights in registers, in the thin
//     kernel's fragment layout (blob of vkhip_conv_pack_weights for thin tile 45); biases seed the
//     accumulators; each value is rounded to fp16 as the conv's own store would, positions outside
//     the conv image hold -inf (the pool's padding);
//   * the pool takes packed fp16 maxima over the LDS tile (exact: the result is bit-identical to
//     the conv launch followed by the pool launch) and stores 8-byte NC4HW4 slots.
// Reference semantics: ConvCpu (src/backend/cpu/ops/conv.cpp:9-92) then the max pool
// (src/backend/cpu/ops/pool.cpp).
#include "conv_kernels.h"

#include <algorithm>
#include <cstring>
#include <mutex>
#include <vector>

namespace vkhip {

    struct ThinPoolArgs {
        const uint2  *x;
        uint2        *y;
        const half_t *w;    // thin fragment layout [m_frag][step][lane][8 halves]
        const float  *bias; // [64]
        int           N, H, W;    // input
        int           OH, OW;     // conv output
        int           POH, POW;   // pooled output
        int           pw;         // pooled columns per item
        int           Cout, cbo;  // channels, channel slots stored
        unsigned      x_bytes, y_bytes;
        int           act;
        float         lo, hi;
    };

    namespace tpl {
        constexpr int PR    = 2;             // pooled rows per item
        constexpr int MAXPW = 28;            // pooled columns per item, at most
        constexpr int CR    = 2 * PR + 1;    // conv rows per item
        constexpr int MCC   = 2 * MAXPW + 1; // conv columns per item, at most
        constexpr int BR    = 2 * (CR - 1) + 7; // input band rows
        constexpr int MBPR  = MCC + 3;       // band pixel pairs per row, at most
        constexpr int MT    = 4;             // 16-channel fragments (64 channels)
        constexpr int NSTEP = 7;             // 49 taps x 4 channels in 32-deep steps
    } // namespace tpl

    __device__ __forceinline__ int tp_div(int v, float r) { return (int) (((float) v + 0.5f) * r); } // v / d, 0 <= v < 2^12, d <= 128

    template <int ACT>
    __global__ __launch_bounds__(256, 2) void conv_thin_pool_kernel(ThinPoolArgs a) {
        using namespace tpl;
        typedef _Float16 half2v __attribute__((ext_vector_type(2)));
        constexpr int NI    = (BR * MBPR + 63) / 64;
        constexpr int BAND  = NI * 1024;
        constexpr int TILE  = MT * 4 * CR * MCC * 8; // 16 slots
        constexpr int DUMPO = BAND + TILE;           // 64 lanes x 8 bytes for lanes past the tile
        static_assert(DUMPO + 512 <= 160 * 1024 / 3, "three workgroups per CU");
        __shared__ __attribute__((aligned(16))) unsigned char sm[DUMPO + 512];
        unsigned char *band = sm;
        unsigned char *tile = sm + BAND;

        const int lane = threadIdx.x & 63;
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int g = lane >> 4, px = lane & 15;
        const int pw = a.pw, cc = 2 * pw + 1, bppr = cc + 3, bc = 2 * bppr;
        const int tp = BR * bppr;      // band pixel pairs
        const int cp = CR * cc;        // conv pixels per slot
        const int pp = PR * pw;        // pooled pixels per slot
        const float rcc = 1.f / (float) cc, rpw = 1.f / (float) pw, rbppr = 1.f / (float) bppr, rpp = 1.f / (float) pp;
        const int rblk = (a.POH + PR - 1) / PR, cblk = (a.POW + pw - 1) / pw;
        const int items = a.N * rblk * cblk;
        constexpr unsigned kInvalid = 0x80000000u;
        const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void *) a.x, (short) 0, (int) a.x_bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t yrs = __builtin_amdgcn_make_buffer_rsrc((void *) a.y, (short) 0, (int) a.y_bytes, 0x00020000);

        half8 wf[MT][NSTEP];
        {
            const half8 *wp = reinterpret_cast<const half8 *>(a.w);
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int j = 0; j < NSTEP; ++j) wf[m][j] = wp[(m * NSTEP + j) * 64 + lane];
        }
        float4v bsv[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) bsv[m] = *reinterpret_cast<const float4v *>(a.bias + (m * 4 + g) * 4);
        // B operand: k = tap*4 + c; the lane's two 4-channel halves of step j are taps 8j + 2g + q
        int  aoff[NSTEP][2];
        bool aval[NSTEP][2];
#pragma unroll
        for (int j = 0; j < NSTEP; ++j)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int tap = 8 * j + 2 * g + q;
                aval[j][q]    = tap < 49;
                aoff[j][q]    = tap < 49 ? (tap / 7) * bc + tap % 7 : 0;
            }

        // items: XCD-contiguous ranges (workgroup b runs on XCD b % 8)
        const int G = gridDim.x;
        const int xcd = blockIdx.x & 7, lb = blockIdx.x >> 3;
        const int gx  = (G >> 3) + ((G & 7) > xcd ? 1 : 0);
        const int pxc = xcd * (G >> 3) + min(xcd, G & 7);
        const int i0  = (int) ((long long) items * pxc / G) + lb;
        const int i1  = (int) ((long long) items * (pxc + gx) / G);
        // band row r, column c of item it <-> input (4 py0 - 5 + r, 4 px0 - 6 + c)
        auto copy_band = [&](int it) __attribute__((always_inline)) {
            const int cb = it % cblk, rest = it / cblk;
            const int px0 = cb * pw, py0 = (rest % rblk) * PR, n = rest / rblk;
            const int iy0 = 4 * py0 - 5, ix0 = 4 * px0 - 6;
#pragma unroll
            for (int r = 0; r < (NI + 3) / 4; ++r) {
                const int i = r * 4 + wave;
                if (i >= NI) break; // wave-uniform
                const int  p   = i * 64 + lane;
                const int  row = tp_div(p, rbppr), pc = p - row * bppr;
                const int  iy  = iy0 + row, ix = ix0 + 2 * pc;
                const bool ok  = (p < tp) & ((unsigned) iy < (unsigned) a.H) & ((unsigned) ix < (unsigned) a.W);
                const unsigned off = ok ? (unsigned) (((n * a.H + iy) * a.W + ix) * 8) : kInvalid;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (__attribute__((address_space(3))) void *) (band + i * 1024), 16, off, 0, 0, 0);
            }
        };
        if (i0 < i1) copy_band(i0);
        for (int it = i0; it < i1; it += gx) {
            const int cb = it % cblk, rest = it / cblk;
            const int px0 = cb * pw, py0 = (rest % rblk) * PR, n = rest / rblk;
            __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); // this wave's copies (and last item's stores) done
            __asm__ volatile("s_barrier" ::: "memory");        // every wave's copies landed
            // conv: tile pixel q = r * cc + c <-> conv output (2 py0 - 1 + r, 2 px0 - 1 + c), window at band row 2r, column 2c + 1
            for (int u = wave; u * 16 < cp; u += 4) {
                const int q = u * 16 + px, r = tp_div(q, rcc), c = q - r * cc;
                const int base = 2 * r * bc + 2 * c + 1;
                float4v   acc[MT];
#pragma unroll
                for (int m = 0; m < MT; ++m) acc[m] = bsv[m];
#pragma unroll
                for (int j = 0; j < NSTEP; ++j) {
                    u32x2 v[2];
#pragma unroll
                    for (int q2 = 0; q2 < 2; ++q2) {
                        const u32x2 t = *reinterpret_cast<const u32x2 *>(band + (base + aoff[j][q2]) * 8);
                        v[q2]         = aval[j][q2] ? t : u32x2 {0u, 0u};
                    }
                    const half8 bf = __builtin_bit_cast(half8, u32x4_make(v[0].x, v[0].y, v[1].x, v[1].y));
#pragma unroll
                    for (int m = 0; m < MT; ++m) acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[m][j], bf, acc[m], 0, 0, 0);
                }
                const int  cy = 2 * py0 - 1 + r, cx = 2 * px0 - 1 + c;
                const bool in = ((unsigned) cy < (unsigned) a.OH) & ((unsigned) cx < (unsigned) a.OW);
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const int oc = (m * 4 + g) * 4;
                    float4v   v  = acc[m];
                    v.x = apply_act(v.x, ACT >= 0 ? ACT : a.act, a.lo, a.hi);
                    v.y = apply_act(v.y, ACT >= 0 ? ACT : a.act, a.lo, a.hi);
                    v.z = apply_act(v.z, ACT >= 0 ? ACT : a.act, a.lo, a.hi);
                    v.w = apply_act(v.w, ACT >= 0 ? ACT : a.act, a.lo, a.hi);
                    if (oc + 0 >= a.Cout) v.x = 0.f;
                    if (oc + 1 >= a.Cout) v.y = 0.f;
                    if (oc + 2 >= a.Cout) v.z = 0.f;
                    if (oc + 3 >= a.Cout) v.w = 0.f;
                    const int o = q < cp ? BAND + ((m * 4 + g) * cp + q) * 8 : DUMPO + lane * 8;
                    *reinterpret_cast<u32x2 *>(sm + o) = in ? __builtin_bit_cast(u32x2, f4_to_h4(v)) : u32x2 {0xFC00FC00u, 0xFC00FC00u};
                }
            }
            // the tile is complete and the band read: the next item's band streams in under the pool
            __builtin_amdgcn_s_waitcnt(0xC07F);
            __asm__ volatile("s_barrier" ::: "memory");
            if (it + gx < i1) copy_band(it + gx);
            // pool: pooled pixel p = pr * pw + pc of slot s, window at tile rows 2 pr .. 2 pr + 2, columns 2 pc .. 2 pc + 2
            for (int i = threadIdx.x; i < MT * 4 * pp; i += 256) {
                const int s = tp_div(i, rpp), p = i - s * pp;
                const int pr = tp_div(p, rpw), pc = p - pr * pw;
                const unsigned char *src = tile + (s * cp + 2 * pr * cc + 2 * pc) * 8;
                // mm[h]: channels 2h, 2h + 1 of the slot
                half2v mm[2];
                mm[0] = mm[1] = __builtin_bit_cast(half2v, 0xFC00FC00u);
#pragma unroll
                for (int dy = 0; dy < 3; ++dy)
#pragma unroll
                    for (int dx = 0; dx < 3; ++dx) {
                        const uint2 t = *reinterpret_cast<const uint2 *>(src + (dy * cc + dx) * 8);
                        mm[0] = __builtin_elementwise_max(mm[0], __builtin_bit_cast(half2v, t.x));
                        mm[1] = __builtin_elementwise_max(mm[1], __builtin_bit_cast(half2v, t.y));
                    }
                const int      py = py0 + pr, pxo = px0 + pc;
                const bool     ok = (py < a.POH) & (pxo < a.POW) & (s < a.cbo);
                const unsigned off = ok ? (unsigned) ((((n * a.cbo + s) * a.POH + py) * a.POW + pxo) * 8) : kInvalid;
                u32x2 o2;
                o2.x = __builtin_bit_cast(unsigned, mm[0]);
                o2.y = __builtin_bit_cast(unsigned, mm[1]);
                __builtin_amdgcn_raw_buffer_store_b64(o2, yrs, off, 0, kStreamStore);
            }
            // no barrier here: the next item's conv writes the tile after the barrier at the loop
            // top, which every wave reaches after its pool reads
        }
    }

    typedef void (*ThinPoolFn)(ThinPoolArgs);

    bool thin_pool_ok(const vkhip_conv_desc *d, const vkhip_conv_plan *plan, const vkhip_pool_desc *p) {
        if (!d || !plan || !p) return false;
        if (plan->algo != VKHIP_CONV_GEMM || plan->tile != 45) return false;
        const bool conv = d->group == 1 && d->Cin > 0 && d->Cin <= 4 && d->Cout > 0 && d->Cout <= 64 && d->KH == 7 && d->KW == 7 && d->SH == 2 &&
                          d->SW == 2 && d->PT == 3 && d->PL == 3 && d->DH == 1 && d->DW == 1 && !d->has_res && !d->in_scale && d->N > 0 &&
                          d->W % 2 == 0 && d->OH == (d->H - 1) / 2 + 1 && d->OW == (d->W - 1) / 2 + 1;
        const bool pool = p->N == d->N && p->C == d->Cout && p->H == d->OH && p->W == d->OW && p->KH == 3 && p->KW == 3 && p->SH == 2 &&
                          p->SW == 2 && p->PT == 1 && p->PL == 1 && p->OH == (d->OH - 1) / 2 + 1 && p->OW == (d->OW - 1) / 2 + 1;
        return conv && pool && (int64_t) d->N * d->H * d->W * 8 < (1LL << 31) && (int64_t) d->N * 16 * p->OH * p->OW * 8 < (1LL << 31);
    }

    int thin_pool_launch(const vkhip_conv_desc *d, const vkhip_pool_desc *p, const void *x, const void *blob, void *y, vkhip_stream_t s) {
        ThinPoolArgs a;
        std::memset(&a, 0, sizeof(a));
        a.x    = (const uint2 *) x;
        a.y    = (uint2 *) y;
        a.bias = (const float *) blob;                                   // [64] fp32
        a.w    = (const half_t *) ((const char *) blob + 64 * 4);       // at align256(64 * 4)
        a.N = d->N; a.H = d->H; a.W = d->W; a.OH = d->OH; a.OW = d->OW; a.POH = p->OH; a.POW = p->OW;
        const int cblk = (int) ceil_div(p->OW, tpl::MAXPW);
        a.pw   = (int) ceil_div(p->OW, cblk);
        a.Cout = d->Cout;
        a.cbo  = (int) ceil_div(d->Cout, 4);
        a.x_bytes = (unsigned) ((int64_t) d->N * d->H * d->W * 8);
        a.y_bytes = (unsigned) ((int64_t) d->N * a.cbo * p->OH * p->OW * 8);
        a.act = d->act; a.lo = d->act_lo; a.hi = d->act_hi;
        ThinPoolFn fn = d->act == VKHIP_ACT_RELU ? conv_thin_pool_kernel<VKHIP_ACT_RELU> : conv_thin_pool_kernel<-1>;
        const int64_t items = (int64_t) d->N * ceil_div(p->OH, tpl::PR) * cblk;
        static std::mutex                                mu;
        static std::vector<std::pair<const void *, int>> occ;
        int per_cu = 0, cus = 256;
        {
            std::lock_guard<std::mutex> lock(mu);
            for (auto &e: occ)
                if (e.first == (const void *) fn) per_cu = e.second;
            if (!per_cu) {
                if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void *) fn, 256, 0) != hipSuccess || per_cu <= 0) per_cu = 1;
                occ.emplace_back((const void *) fn, per_cu);
            }
            int dev = 0;
            if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
        }
        const int64_t grid = std::max<int64_t>(1, std::min<int64_t>((int64_t) cus * per_cu, items));
        fn<<<dim3((unsigned) grid), 256, 0, resolve_stream(s)>>>(a);
        return check_launch("conv_thin_pool");
    }

} // namespace vkhip
