/* r3d_gemv_layout.h -- LDS layout of the decode GEMV's per-run buffers (shared by the
 * kernel and the host code that sizes its workgroups).  Pure C++. */
#ifndef R3D_GEMV_LAYOUT_H
#define R3D_GEMV_LAYOUT_H

#include "r3d_plan.h"

namespace r3d {

constexpr int kRunBytes = 512;               /* weight bytes of one row per run */
constexpr int kPairPitch = 2 * kRunBytes + 16;

template <int ENC, int MT>
struct GemvLayout {
    static constexpr int SB = ENC == ENC_MXFP4A8 ? 64 : 128;       /* weight bytes per step */
    static constexpr int RS = kRunBytes / SB;                        /* steps per run */
    static constexpr int DB = MT <= 4 ? 2 : 1;                       /* run buffers per wave */
    static constexpr int W = 0;                                      /* 8 row pairs */
    static constexpr int AC = W + 8 * kPairPitch;                    /* MT rows of 1040 */
    static constexpr int SC = AC + MT * 1040;                        /* weight scales */
    static constexpr int N_SC = ENC == ENC_MXFP4A8 ? 2 : 1;          /* 256 B / 128 B each */
    static constexpr int AS = SC + N_SC * 256;                       /* a_scale [MT][RS] f32 */
    static constexpr int N_AS = (MT * RS * 4 + 255) / 256;           /* 256 B each */
    static constexpr int BUF = AS + N_AS * 256;                      /* one run buffer */
    static constexpr int WAVE = DB * BUF;
    /* direct-load instructions per run: weights, activations, weight scales, a_scales */
    static constexpr int LOADS = 8 + MT + N_SC + N_AS;
};

/* LDS bytes one decode wave needs (host side: picks waves per workgroup). */
inline int gemv_wave_lds(int enc, int mt) {
    if (enc == ENC_MXFP4A8)
        return mt == 1 ? GemvLayout<ENC_MXFP4A8, 1>::WAVE
             : mt == 4 ? GemvLayout<ENC_MXFP4A8, 4>::WAVE : GemvLayout<ENC_MXFP4A8, 16>::WAVE;
    return mt == 1 ? GemvLayout<ENC_FP8A8, 1>::WAVE
         : mt == 4 ? GemvLayout<ENC_FP8A8, 4>::WAVE : GemvLayout<ENC_FP8A8, 16>::WAVE;
}

}  // namespace r3d

#endif /* R3D_GEMV_LAYOUT_H */
