/* r3d_prefill_layout.h -- LDS ring of the mxfp4 prefill GEMM (shared by the kernel and
 * the host code that picks its tile).  Pure C++. */
#ifndef R3D_PREFILL_LAYOUT_H
#define R3D_PREFILL_LAYOUT_H

namespace r3d {

enum PrefillMode { PF_A8 = 0, PF_MX8 = 1 };

/* One ring stage holds everything a 128-wide K step of a BN x BM tile reads, and LOADS
 * is the number of direct-load instructions each of the 4 waves issues per stage. */
template <int WNF, int WMF, int NST>
struct PrefillLayout {
    static constexpr int BN = 32 * WNF;           /* weight rows per tile: 2 waves x WNF frags */
    static constexpr int BM = 32 * WMF;           /* tokens per tile: 2 waves x WMF frags */
    static constexpr int WFR = 2 * WNF;           /* 16-row weight fragments per tile */
    static constexpr int WLD = (WFR + 3) / 4;     /* weight loads per wave per step */
    static constexpr int ALD = BM / 32;           /* activation loads per wave per step */
    static constexpr int W = 0;                   /* [4 WLD][1 KB] weight fragments (+ pad) */
    static constexpr int S = W + 4 * WLD * 1024;  /* [256] dwords: 4 E8M0 per weight row */
    static constexpr int A = S + 1024;            /* [BM/16][2 halves][1 KB] activations */
    static constexpr int AS = A + BM * 128;       /* [256] dwords: 4 E8M0 or one f32 per token */
    static constexpr int STAGE = AS + 1024;
    static constexpr int LDS = NST * STAGE;
    static constexpr int LOADS = WLD + 1 + ALD + 1;
    static_assert(BN <= 256 && BM <= 256, "one scale load per wave covers 256 rows");
    static_assert(LDS <= 160 * 1024, "ring exceeds the CU's LDS");
};

/* Host mirror of PrefillLayout::STAGE for any (wnf, wmf). */
constexpr int prefill_stage_bytes(int wnf, int wmf) {
    return 4 * ((2 * wnf + 3) / 4) * 1024 + 1024 + 32 * wmf * 128 + 1024;
}

}  // namespace r3d

#endif /* R3D_PREFILL_LAYOUT_H */
