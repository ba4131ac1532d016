/* r3d_prefill_layout.h -- LDS ring of the prefill GEMM (shared by the kernel and the host
 * code that picks its tile).  Pure C++. */
#ifndef R3D_PREFILL_LAYOUT_H
#define R3D_PREFILL_LAYOUT_H

namespace r3d {

enum PrefillMode { PF_A8 = 0, PF_MX8 = 1, PF_F8 = 2 };

/* A workgroup is 8 waves (two per SIMD): 2 along N, each WNF 16-row weight fragments,
 * by 4 along M, each WMW 16-token fragments.  One ring stage holds everything a 128-wide
 * K step of the BN x BM tile reads, and LOADS is the number of direct-load instructions
 * each wave issues per stage (the same for every wave, so the vmcnt bookkeeping is
 * uniform).  WH is the number of 1 KB plane images per weight fragment: 1 for e2m1 (16
 * rows x 64 bytes), 2 for e4m3 (16 rows x 128 bytes, two 64-byte halves, like the
 * activation fragments). */
template <int WNF, int WMW, int NST, int WH = 1>
struct PrefillLayout {
    static constexpr int WAVES = 8;
    static constexpr int BN = 32 * WNF;           /* weight rows per tile */
    static constexpr int BM = 64 * WMW;           /* tokens per tile */
    static constexpr int WFR = 2 * WNF;           /* 16-row weight fragments per tile */
    static constexpr int WLD = (WH * WFR + 7) / 8;   /* weight loads per wave per step */
    static constexpr int ALD = BM / 64;           /* activation loads per wave per step */
    static constexpr int W = 0;                   /* [8 WLD][1 KB] weight images (+ pad) */
    static constexpr int S = W + 8 * WLD * 1024;  /* [256] dwords per weight row: 4 E8M0
                                                     (e2m1) or one bf16 scale (e4m3) */
    static constexpr int A = S + 1024;            /* [BM/16][2 halves][1 KB] activations */
    static constexpr int AS = A + BM * 128;       /* [256] dwords: 4 E8M0 or one f32 per token */
    static constexpr int STAGE = AS + 1024;
    static constexpr int LDS = NST * STAGE;
    static constexpr int LOADS = WLD + ALD + 1;   /* + one scale load (weights or tokens) */
    static_assert(BN <= 256 && BM <= 256, "four scale loads of 64 rows cover a tile side");
    static_assert(LDS <= 160 * 1024, "ring exceeds the CU's LDS");
};

/* Host mirror of PrefillLayout::STAGE for any (wnf, wmw, wh). */
constexpr int prefill_stage_bytes(int wnf, int wmw, int wh = 1) {
    return 8 * ((wh * 2 * wnf + 7) / 8) * 1024 + 1024 + 64 * wmw * 128 + 1024;
}

}  // namespace r3d

#endif /* R3D_PREFILL_LAYOUT_H */
