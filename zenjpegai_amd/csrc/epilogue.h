// Fused epilogue of the convolution kernels (conv.hip, conv32.hip): activation, residual
// operation, pixel shuffle, denormalisation, tile-core windows, chroma decimation and
// quantisation, each as separate IEEE operations in f32.
#pragma once

#include "conv.h"

namespace zjai {

__device__ __forceinline__ float apply_act(int act, float v) {
    if (act == ACT_RELU) return fmaxf(v, 0.0f);
    if (act == ACT_LEAKY) return v < 0.0f ? v * 0.01f : v;
    if (act == ACT_SIGMOID) return sigmoidf_ref(v);
    return v;
}

// v / s and v % s for a subsampling factor s (uniform per launch; 1 and 2 without a division).
// v >= 0 wherever the quotient is used; for v < 0 only whether the remainder is zero matters.
__device__ __forceinline__ int sub_div(int v, int s) { return s == 1 ? v : s == 2 ? (v >> 1) : v / s; }
__device__ __forceinline__ int sub_rem(int v, int s) { return s == 1 ? 0 : s == 2 ? (v & 1) : v % s; }

// One sample of a planar picture output at plane offset o: denormalise, then f32 or quantised u16.
__device__ __forceinline__ void plane_store(const ConvParams& p, long long o, float s) {
    if (p.denorm) {
        s = s * 128.0f;
        s = s + 127.5f;
        s = s < 0.0f ? 0.0f : s;
        s = s > 255.0f ? 255.0f : s;
    }
    if (p.bit_depth == 0) {
        ((float*)p.plane)[o] = s;
    } else {
        // quantize_plane (src/decoder/output.rs:330-342): rint(clamp(x,0,255)/255*max).
        const float mx = (float)((1u << p.bit_depth) - 1u);
        float q = s < 0.0f ? 0.0f : s;
        q = q > 255.0f ? 255.0f : q;
        q = q / 255.0f;
        q = q * mx;
        q = rintf(q);
        q = q < 0.0f ? 0.0f : q;
        q = q > mx ? mx : q;
        ((uint16_t*)p.plane)[o] = (uint16_t)q;
    }
}

template <typename T>
__device__ __forceinline__ void epilogue_store(const ConvParams& p, int b, int oy, int ox, int oc0,
                                               int nvalid, f32x4 v) {
    // Activation, then the residual operation, each as separate IEEE operations.
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = apply_act(p.act, v[i]);
    if (p.res != RES_NONE) {
        const long long o1 = (long long)b * p.r1.bstride + (long long)oy * p.r1.row +
                             (long long)ox * p.r1.cs + p.r1.c_off + oc0;
        f32x4 r1;
        if (nvalid == 4) {
            r1 = load4<T>((const T*)p.r1.p + o1);
        } else {
            for (int i = 0; i < 4; ++i) r1[i] = i < nvalid ? to_f32(((const T*)p.r1.p)[o1 + i]) : 0.0f;
        }
        if (p.res == RES_ADD) {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = v[i] + r1[i];
        } else if (p.res == RES_GATE) {
#pragma unroll
            for (int i = 0; i < 4; ++i) { const float g = 1.0f + v[i]; v[i] = r1[i] * g; }
        } else if (p.res == RES_MUL) {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = r1[i] * v[i];
        } else if (p.res == RES_CAB) {
            const long long o2 = (long long)b * p.r2.bstride + (long long)oy * p.r2.row +
                                 (long long)ox * p.r2.cs + p.r2.c_off + oc0;
            f32x4 r2;
            if (nvalid == 4) {
                r2 = load4<T>((const T*)p.r2.p + o2);
            } else {
                for (int i = 0; i < 4; ++i) r2[i] = i < nvalid ? to_f32(((const T*)p.r2.p)[o2 + i]) : 0.0f;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float s = sigmoidf_ref(v[i]);
                const float t = r1[i] * s;
                v[i] = t + r2[i];
            }
        }
    }
    if (p.out_mode == OUT_NHWC) {
        T* y = (T*)p.y.p + (long long)b * p.y.bstride;
        if (p.ps == 1) {
            const long long o = (long long)oy * p.y.row + (long long)ox * p.y.cs + p.y.c_off + oc0;
            if (nvalid == 4) {
                store4<T>(y + o, v);
            } else {
                for (int i = 0; i < nvalid; ++i) y[o + i] = from_f32<T>(v[i]);
            }
        } else {
            const int r = p.ps, rr = r * r;
            for (int i = 0; i < nvalid; ++i) {
                const int oc = oc0 + i, c = oc / rr, sub = oc - c * rr;
                const int Y = oy * r + sub / r, X = ox * r + sub % r;
                y[(long long)Y * p.y.row + (long long)X * p.y.cs + p.y.c_off + c] = from_f32<T>(v[i]);
            }
        }
        return;
    }
    // Planar picture output (last layer): pixel shuffle, denormalise, crop to the kept window,
    // chroma subsampling, f32 or quantised u16.
    const int r = p.ps, rr = r * r;
    if (r == 1) {
        // No pixel shuffle: the nvalid channels share one output pixel, so its subsampling and
        // window tests and plane offset are computed once (the subsampling test first: with
        // 4:2:0 planes it drops three of every four pixels, often a whole wave's).
        const int wy = oy - p.win_y0[b], wx = ox - p.win_x0[b];
        const int py = p.dst_y0[b] + wy, px = p.dst_x0[b] + wx;
        if (sub_rem(py, p.sv) || sub_rem(px, p.sh)) return;
        if (wy < 0 || wy >= p.win_h[b] || wx < 0 || wx >= p.win_w[b]) return;
        const long long o0 = (long long)sub_div(py, p.sv) * p.pl_row + sub_div(px, p.sh);
        for (int i = 0; i < nvalid; ++i) plane_store(p, (long long)(oc0 + i) * p.pl_cstride + o0, v[i]);
        return;
    }
    for (int i = 0; i < nvalid; ++i) {
        const int oc = oc0 + i, c = oc / rr, sub = oc - c * rr;
        const int Y = oy * r + sub / r, X = ox * r + sub % r;
        const int wy = Y - p.win_y0[b], wx = X - p.win_x0[b];
        if (wy < 0 || wy >= p.win_h[b] || wx < 0 || wx >= p.win_w[b]) continue;
        const int py = p.dst_y0[b] + wy, px = p.dst_x0[b] + wx;
        if (py % p.sv || px % p.sh) continue;
        plane_store(p, (long long)c * p.pl_cstride + (long long)(py / p.sv) * p.pl_row + px / p.sh, v[i]);
    }
}

// True when a launch's epilogue is an NHWC store without pixel shuffle: epilogue_store8 (any
// activation and residual operation) covers it.
__device__ __forceinline__ bool epilogue_simple(const ConvParams& p) {
    return p.out_mode == OUT_NHWC && p.ps == 1;
}

// NHWC output with a pixel shuffle by 2 and no residual operation: epilogue_store_ps2 applies.
__device__ __forceinline__ bool epilogue_ps2(const ConvParams& p) {
    return p.out_mode == OUT_NHWC && p.ps == 2 && p.res == RES_NONE;
}

// epilogue_store for the pixel shuffle by 2 when epilogue_ps2 holds, four output channels at a
// time: output channels c .. c + 3 at sub-position s of position (oy, ox) take conv channels
// 4 c + s, 4 (c + 1) + s, .. (v in that order); the activation per element, then one vector
// store of the four (epilogue_store writes the same values one channel at a time).
template <typename T>
__device__ __forceinline__ void epilogue_store_ps2(const ConvParams& p, int b, int oy, int ox, int s, int c,
                                                   f32x4 v) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = apply_act(p.act, v[i]);
    T* y = (T*)p.y.p + (long long)b * p.y.bstride;
    const int Y = 2 * oy + (s >> 1), X = 2 * ox + (s & 1);
    store4<T>(y + (long long)Y * p.y.row + (long long)X * p.y.cs + p.y.c_off + c, v);
}

// epilogue_store for 8 consecutive channels of one position (all valid) when epilogue_simple
// holds: the same IEEE operations in the same order, one 16-byte (16-bit types) or two 16-byte
// (f32) stores, 8-channel residual loads.
template <typename T>
__device__ __forceinline__ void epilogue_store8(const ConvParams& p, int b, int oy, int ox, int oc0, f32x4 v0,
                                                f32x4 v1) {
    float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
    if (p.act == ACT_RELU) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = fmaxf(v[i], 0.0f);
    } else if (p.act == ACT_LEAKY) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = v[i] < 0.0f ? v[i] * 0.01f : v[i];
    } else if (p.act == ACT_SIGMOID) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = sigmoidf_ref(v[i]);
    }
    if (p.res != RES_NONE) {
        const T* r = (const T*)p.r1.p + (long long)b * p.r1.bstride + (long long)oy * p.r1.row +
                     (long long)ox * p.r1.cs + p.r1.c_off + oc0;
        const f32x4 ra = load4<T>(r), rb = load4<T>(r + 4);
        const float rv[8] = {ra[0], ra[1], ra[2], ra[3], rb[0], rb[1], rb[2], rb[3]};
        if (p.res == RES_ADD) {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = v[i] + rv[i];
        } else if (p.res == RES_GATE) {
#pragma unroll
            for (int i = 0; i < 8; ++i) { const float g = 1.0f + v[i]; v[i] = rv[i] * g; }
        } else if (p.res == RES_MUL) {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = rv[i] * v[i];
        } else {  // RES_CAB: r1 * sigmoid(v) + r2
            const T* r2 = (const T*)p.r2.p + (long long)b * p.r2.bstride + (long long)oy * p.r2.row +
                          (long long)ox * p.r2.cs + p.r2.c_off + oc0;
            const f32x4 sa = load4<T>(r2), sb = load4<T>(r2 + 4);
            const float sv[8] = {sa[0], sa[1], sa[2], sa[3], sb[0], sb[1], sb[2], sb[3]};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float sg = sigmoidf_ref(v[i]);
                const float t = rv[i] * sg;
                v[i] = t + sv[i];
            }
        }
    }
    T* y = (T*)p.y.p + (long long)b * p.y.bstride + (long long)oy * p.y.row + (long long)ox * p.y.cs + p.y.c_off + oc0;
    store4<T>(y, f32x4{v[0], v[1], v[2], v[3]});
    store4<T>(y + 4, f32x4{v[4], v[5], v[6], v[7]});
}

}  // namespace zjai
