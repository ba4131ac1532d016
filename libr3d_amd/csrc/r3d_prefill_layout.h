/* r3d_prefill_layout.h -- LDS ring of the prefill GEMM (shared by the kernel and the host
 * code that picks its tile).  Pure C++. */
#ifndef R3D_PREFILL_LAYOUT_H
#define R3D_PREFILL_LAYOUT_H

namespace r3d {

enum PrefillMode { PF_A8 = 0, PF_MX8 = 1, PF_F8 = 2 };

/* A workgroup is WV waves: 2 along N, each WNF 16-row weight fragments, by WV / 2 along M,
 * each WMW 16-token fragments -- 8 waves (two per SIMD), or 4 (one per SIMD, twice the
 * registers a wave, for tiles whose operands and results do not fit 256).  One ring stage
 * holds everything a 128-wide K step of the BN x BM tile reads, and LOADS is the number of
 * direct-load instructions each wave issues per stage (the same for every wave, so the
 * vmcnt bookkeeping is uniform).  WH is the number of 1 KB plane images per weight
 * fragment: 1 for e2m1 (16 rows x 64 bytes), 2 for e4m3 (16 rows x 128 bytes, two 64-byte
 * halves, like the activation fragments).  Scales: at 8 waves, waves 0-3 fetch the weight
 * rows' and waves 4-7 the tokens' (one load each); at 4 waves every wave fetches 64 of
 * each (two loads). */
template <int WNF, int WMW, int NST, int WH = 1, int WV = 8>
struct PrefillLayout {
    static_assert(WV == 8 || WV == 4, "8 or 4 waves a workgroup");
    static constexpr int WAVES = WV;
    static constexpr int BN = 32 * WNF;           /* weight rows per tile */
    static constexpr int BM = 8 * WV * WMW;       /* tokens per tile */
    static constexpr int WFR = 2 * WNF;           /* 16-row weight fragments per tile */
    static constexpr int WLD = (WH * WFR + WV - 1) / WV;   /* weight loads per wave per step */
    static constexpr int ALD = 2 * (BM / 16) / WV;          /* activation loads per wave per step */
    static constexpr int SLD = WV == 8 ? 1 : 2;   /* scale loads per wave per step */
    static constexpr int W = 0;                   /* [WV WLD][1 KB] weight images (+ pad) */
    static constexpr int S = W + WV * WLD * 1024; /* [256] dwords per weight row: 4 E8M0
                                                     (e2m1) or one bf16 scale (e4m3) */
    static constexpr int A = S + 1024;            /* [BM/16][2 halves][1 KB] activations */
    static constexpr int AS = A + BM * 128;       /* [256] dwords: 4 E8M0 or one f32 per token */
    static constexpr int STAGE = AS + 1024;
    static constexpr int LDS = NST * STAGE;
    static constexpr int LOADS = WLD + ALD + SLD;
    static_assert(BN <= 256 && BM <= 256, "four scale loads of 64 rows cover a tile side");
    static_assert(LDS <= 160 * 1024, "ring exceeds the CU's LDS");
};

/* Host mirror of PrefillLayout::STAGE for any (wnf, wmw, wh, wv). */
constexpr int prefill_stage_bytes(int wnf, int wmw, int wh = 1, int wv = 8) {
    return wv * ((wh * 2 * wnf + wv - 1) / wv) * 1024 + 1024 + 8 * wv * wmw * 128 + 1024;
}

}  // namespace r3d

#endif /* R3D_PREFILL_LAYOUT_H */
