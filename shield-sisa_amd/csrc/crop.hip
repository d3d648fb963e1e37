// Face crops on the GPU: the reference's lazy native crop (engine/preprocess/canvas.cpp:66-91, shv_prep.h:181-186)
//   crop = cv2.resize(canvas[4y:4(y+h), 4x:4(x+w)], (320, 180), INTER_AREA)
// where canvas is the native frame resized into 1280x720 (INTER_AREA when shrinking, INTER_LINEAR when enlarging,
// letterbox bars zero; engine/preprocess/geometry.cpp:77-88).  Every output byte is a fixed function of a small
// source neighbourhood, so each is computed independently: a patch kernel evaluates the canvas pixels a crop needs
// (only those) into a scratch buffer, a crop kernel resizes the patch to 320x180.
//
// The resize arithmetic is OpenCV 4.13's for 8-bit images, as the reference restates it in
// engine/preprocess/cvresize.cpp:
//   area, general scale (cvresize.cpp:22-38, 303-335, 421-447): per output, for each source row of its area tab in
//     order: t = ((0 + S0 a0) + S1 a1) + ... over the column taps, sum = b0 t0 (first row) then sum + b_j t_j;
//     out = saturate(rint(sum)); every float operation rounded separately;
//   area, integer scale (cvresize.cpp:612-666): 2x2 blocks (S00 + S01 + S10 + S11 + 2) >> 2, other full blocks
//     rint((float)sum * (1.f / (ix iy))), partial blocks rint((float)sum / count), past the source 0;
//   linear, 11-bit fixed point (cvresize.cpp:185-212, 668-719): h = S[x] a0 + S[x+1] a1 (or S[x] 2048 past lxmax),
//     out = (((b0 (h0 >> 4)) >> 16) + ((b1 (h1 >> 4)) >> 16) + 2) >> 2, rows clipped into the source;
//   equal sizes: copy.
// The plan tables (taps, weights, coefficients) are built on the host in the same double / float arithmetic.
// I420 frames are converted per native pixel as the reference does row by row (engine/preprocess/color.cpp:4-11,
// 57-109: ffmpeg's unscaled yuv420p -> rgb24, BT.601 limited range, 16-bit fixed point, chroma of (x, y) at
// [y / 2][x / 2]).
#include "dev_common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

namespace shv {
namespace {

#define CROP_CHECK(expr)                                                                                     \
    do {                                                                                                     \
        const hipError_t err__ = (expr);                                                                     \
        if (err__ != hipSuccess) throw std::runtime_error(std::string("HIP error ") + hipGetErrorString(err__)); \
    } while (0)

constexpr int CROP_W = 320, CROP_H = 180, COEF_BITS = 11, COEF_SCALE = 1 << COEF_BITS;

// one resize geometry on the device; kind 0 copy, 1 area (general), 2 area (integer scale), 3 linear (11 bit)
struct PlanDev {
    int kind = 0, sw = 0, sh = 0, dw = 0, dh = 0;
    const int *xfirst = nullptr, *xsi = nullptr, *yfirst = nullptr, *ysi = nullptr;   // area taps (pixels)
    const float *xal = nullptr, *yal = nullptr;                                          // area weights
    int ix = 0, iy = 0;
    float fscale = 0.0f;
    const int *lxofs = nullptr, *lalpha = nullptr, *lyofs = nullptr, *lbeta = nullptr;   // linear
    int lxmax = 0;
};

// one crop: its native frame, canvas geometry and patch
struct JobDev {
    const uint8_t* frame;   // RGB, or the I420 Y plane
    long long stride;
    const uint8_t *u, *v;   // I420 chroma planes
    long long u_stride, v_stride;
    long long patch_off;   // byte offset of the patch in the scratch buffer
    int canvas_plan, crop_plan;
    int px0, py0, pw, ph;  // patch = canvas columns px0 .. px0+pw, rows py0 .. py0+ph
    int left, top, new_w, new_h;
};

__device__ __forceinline__ int sat_u8(float v) {
    const float r = __builtin_rintf(v);   // cvRound: round half to even
    return r < 0.0f ? 0 : (r > 255.0f ? 255 : int(r));
}
__device__ __forceinline__ int clip_row(int y, int n) { return y >= 0 ? (y < n ? y : n - 1) : 0; }

// output pixel (dx, dy), all channels c = 0..2, of plan p over a source read as src(x, y, c); the channels are
// independent, each computed with the reference's per-byte operations (taps read once per pixel)
template <class Src>
__device__ __forceinline__ void resize_px3(const PlanDev& p, const Src& src, int dx, int dy, int (&o)[3]) {
    switch (p.kind) {
    case 0:
#pragma unroll
        for (int c = 0; c < 3; ++c) o[c] = 0;
        src.pix(dx, dy, o);
        return;
    case 1: {
        const int ya = p.yfirst[dy], ye = p.yfirst[dy + 1], xa = p.xfirst[dx], xe = p.xfirst[dx + 1];
        float sum[3] = {0.0f, 0.0f, 0.0f};
        for (int j = ya; j < ye; ++j) {
            const int sy = p.ysi[j];
            const float beta = p.yal[j];
            float t[3] = {0.0f, 0.0f, 0.0f};
            for (int k = xa; k < xe; ++k) {
                const float al = p.xal[k];
                int px[3];
                src.pix(p.xsi[k], sy, px);
#pragma unroll
                for (int c = 0; c < 3; ++c) t[c] = t[c] + float(px[c]) * al;
            }
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                const float bt = beta * t[c];
                sum[c] = j == ya ? bt : sum[c] + bt;
            }
        }
#pragma unroll
        for (int c = 0; c < 3; ++c) o[c] = sat_u8(sum[c]);
        return;
    }
    case 2: {
        const int sx0 = dx * p.ix, sy0 = dy * p.iy;
        if (sy0 >= p.sh) {
            o[0] = o[1] = o[2] = 0;
            return;
        }
        if (sy0 + p.iy <= p.sh && dx < p.sw / p.ix) {   // a full block
            int sm[3] = {0, 0, 0};
            for (int r = 0; r < p.iy; ++r)
                for (int q = 0; q < p.ix; ++q) {
                    int px[3];
                    src.pix(sx0 + q, sy0 + r, px);
#pragma unroll
                    for (int c = 0; c < 3; ++c) sm[c] += px[c];
                }
            if (p.ix == 2 && p.iy == 2) {
#pragma unroll
                for (int c = 0; c < 3; ++c) o[c] = (sm[c] + 2) >> 2;
                return;
            }
#pragma unroll
            for (int c = 0; c < 3; ++c) o[c] = sat_u8(float(sm[c]) * p.fscale);
            return;
        }
        if (sx0 >= p.sw) {
            o[0] = o[1] = o[2] = 0;
            return;
        }
        const int nr = min(p.iy, p.sh - sy0);
        int sm[3] = {0, 0, 0}, count = 0;
        for (int r = 0; r < nr; ++r)
            for (int q = 0; q < p.ix && sx0 + q < p.sw; ++q) {
                int px[3];
                src.pix(sx0 + q, sy0 + r, px);
#pragma unroll
                for (int c = 0; c < 3; ++c) sm[c] += px[c];
                ++count;
            }
#pragma unroll
        for (int c = 0; c < 3; ++c) o[c] = sat_u8(float(sm[c]) / float(count));
        return;
    }
    default: {
        const int sx = p.lxofs[dx], a0 = p.lalpha[2 * dx], a1 = p.lalpha[2 * dx + 1];
        const int sy = p.lyofs[dy];
        const int ra = clip_row(sy, p.sh), rb = clip_row(sy + 1, p.sh);
        const bool in = dx < p.lxmax;
        const int b0 = p.lbeta[2 * dy], b1 = p.lbeta[2 * dy + 1];
        const int sx1 = in ? sx + 1 : sx;
        int s00[3], s01[3], s10[3], s11[3];
        src.pix(sx, ra, s00);
        src.pix(sx1, ra, s01);
        src.pix(sx, rb, s10);
        src.pix(sx1, rb, s11);
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            const int h0 = in ? s00[c] * a0 + s01[c] * a1 : s00[c] * COEF_SCALE;
            const int h1 = in ? s10[c] * a0 + s11[c] * a1 : s10[c] * COEF_SCALE;
            o[c] = (((b0 * (h0 >> 4)) >> 16) + ((b1 * (h1 >> 4)) >> 16) + 2) >> 2;
        }
        return;
    }
    }
}

struct FrameSrc {   // native RGB frame
    const uint8_t* f;
    long long stride;
    __device__ void pix(int x, int y, int (&v)[3]) const {
        const uint8_t* q = f + (long long)y * stride + 3 * x;
        v[0] = q[0]; v[1] = q[1]; v[2] = q[2];
    }
};
// BT.601 limited-range coefficients of ffmpeg's yuv2rgb tables (contrast = saturation = 1 << 16, brightness 0),
// rounded to 16 bits as av_clip_int16((x + 2^15) >> 16): Y 76309 (= 65536 * 255 / 219) and the inverse-table
// entries 104597 (V->R), 132201 (U->B), -25675 (U->G), -53279 (V->G), each times 2^13; Y offset 16 << 19
struct Yuv {
    int y_coeff, vr, ub, ug, vg, y_off, uv_off;
};
struct I420Src {   // native I420 frame, converted per pixel
    const uint8_t *Y, *U, *V;
    long long ys, us, vs;
    Yuv k;
    __device__ static int sat16(int v) { return v < -32768 ? -32768 : (v > 32767 ? 32767 : v); }
    __device__ static int mulhi(int a, int b) { return (a * b) >> 16; }
    __device__ static int sat8(int v) { return v < 0 ? 0 : (v > 255 ? 255 : v); }
    __device__ void pix(int x, int y, int (&v)[3]) const {
        const int yp = int(short((int(Y[(long long)y * ys + x]) << 3) - k.y_off));
        const int up = sat16((int(U[(long long)(y >> 1) * us + (x >> 1)]) << 3) - k.uv_off);
        const int vp = sat16((int(V[(long long)(y >> 1) * vs + (x >> 1)]) << 3) - k.uv_off);
        const int yy = mulhi(yp, k.y_coeff);
        const int cg = sat16(mulhi(up, k.ug) + mulhi(vp, k.vg));
        v[0] = sat8(sat16(yy + mulhi(vp, k.vr)));
        v[1] = sat8(sat16(yy + cg));
        v[2] = sat8(sat16(yy + mulhi(up, k.ub)));
    }
};
struct PatchSrc {   // a crop's patch in the scratch buffer
    const uint8_t* p;
    int pw;
    __device__ void pix(int x, int y, int (&v)[3]) const {
        const uint8_t* q = p + ((long long)y * pw + x) * 3;
        v[0] = q[0]; v[1] = q[1]; v[2] = q[2];
    }
};

// One block per (output row, crop): the row's vertical taps are uniform across the block, and its threads walk the
// row's pixels, so source reads and output writes are contiguous across a wave; each thread takes all three channels
// of its pixel (taps read once).

// canvas pixels of each crop's patch (blockIdx.x = patch row, blockIdx.y = crop); bars outside the pasted frame are
// zero
template <bool I420>
__global__ void __launch_bounds__(256)
crop_patch_kernel(const JobDev* __restrict__ jobs, const PlanDev* __restrict__ plans, uint8_t* __restrict__ scratch,
                  Yuv yuv) {
    const JobDev j = jobs[blockIdx.y];
    const int py = blockIdx.x;
    if (py >= j.ph) return;
    uint8_t* d = scratch + j.patch_off + 3LL * j.pw * py;
    const int cy = j.py0 + py - j.top;   // row of the resized frame
    const int n = 3 * j.pw;
    if (cy < 0 || cy >= j.new_h) {
        for (int e = threadIdx.x; e < n; e += 256) d[e] = 0;
        return;
    }
    const PlanDev p = plans[j.canvas_plan];
    const FrameSrc rgb{j.frame, j.stride};
    const I420Src i420{j.frame, j.u, j.v, j.stride, j.u_stride, j.v_stride, yuv};
    for (int px = threadIdx.x; px < j.pw; px += 256) {
        const int cx = j.px0 + px - j.left;
        int v[3] = {0, 0, 0};
        if (cx >= 0 && cx < j.new_w) {
            if constexpr (I420) resize_px3(p, i420, cx, cy, v);
            else resize_px3(p, rgb, cx, cy, v);
        }
        d[3 * px] = uint8_t(v[0]);
        d[3 * px + 1] = uint8_t(v[1]);
        d[3 * px + 2] = uint8_t(v[2]);
    }
}

// 320 x 180 crop of each patch (blockIdx.x = crop row, blockIdx.y = crop)
__global__ void __launch_bounds__(256)
crop_resize_kernel(const JobDev* __restrict__ jobs, const PlanDev* __restrict__ plans,
                   const uint8_t* __restrict__ scratch, uint8_t* __restrict__ out) {
    const JobDev j = jobs[blockIdx.y];
    const int oy = blockIdx.x;
    const PlanDev p = plans[j.crop_plan];
    const PatchSrc src{scratch + j.patch_off, j.pw};
    uint8_t* d = out + (long long)blockIdx.y * (CROP_W * CROP_H * 3) + 3LL * CROP_W * oy;
    for (int ox = threadIdx.x; ox < CROP_W; ox += 256) {
        int v[3];
        resize_px3(p, src, ox, oy, v);
        d[3 * ox] = uint8_t(v[0]);
        d[3 * ox + 1] = uint8_t(v[1]);
        d[3 * ox + 2] = uint8_t(v[2]);
    }
}

// ------------------------------------------------------------------------------------------------ host plans
inline long py_round(double v) { return long(std::nearbyint(v)); }   // Python round(): half to even
inline int rint_f(float v) { return int(std::nearbyintf(v)); }

struct Tap {
    int d, s;
    float w;
};
// OpenCV's area taps for one axis (computeResizeAreaTab): output cell [d scale, (d + 1) scale) of the source,
// partial source pixels weighted by their covered fraction of the cell
std::vector<Tap> area_taps(int ssize, int dsize, double scale) {
    std::vector<Tap> t;
    for (int d = 0; d < dsize; ++d) {
        const double f1 = d * scale, f2 = f1 + scale;
        const double cell = std::min(scale, ssize - f1);
        int s1 = int(std::ceil(f1)), s2 = int(std::floor(f2));
        s2 = std::min(s2, ssize - 1);
        s1 = std::min(s1, s2);
        if (s1 - f1 > 1e-3) t.push_back({d, s1 - 1, float((s1 - f1) / cell)});
        for (int s = s1; s < s2; ++s) t.push_back({d, s, float(1.0 / cell)});
        if (f2 - s2 > 1e-3) t.push_back({d, s2, float(std::min(std::min(f2 - s2, 1.0), cell) / cell)});
    }
    return t;
}

struct PlanHost {
    int kind = 0, sw = 0, sh = 0, dw = 0, dh = 0, ix = 0, iy = 0, lxmax = 0;
    float fscale = 0.0f;
    std::vector<int> xfirst, xsi, yfirst, ysi, lxofs, lalpha, lyofs, lbeta;
    std::vector<float> xal, yal;
};

void index_taps(const std::vector<Tap>& t, int dsize, std::vector<int>& first, std::vector<int>& si,
                std::vector<float>& w) {
    first.assign(size_t(dsize) + 1, int(t.size()));
    for (int k = int(t.size()) - 1; k >= 0; --k) first[size_t(t[size_t(k)].d)] = k;
    for (int d = dsize - 1; d >= 0; --d) first[size_t(d)] = std::min(first[size_t(d)], first[size_t(d) + 1]);
    for (const Tap& x : t) {
        si.push_back(x.s);
        w.push_back(x.w);
    }
}

// interpolation: 1 INTER_LINEAR, 3 INTER_AREA (OpenCV codes); false where the reference has no plan either
bool make_plan(int sw, int sh, int dw, int dh, int interpolation, PlanHost& p) {
    p = PlanHost();
    p.sw = sw; p.sh = sh; p.dw = dw; p.dh = dh;
    if (sw <= 0 || sh <= 0 || dw <= 0 || dh <= 0) return false;
    if (sw == dw && sh == dh) return true;   // copy
    const double inv_x = double(dw) / sw, inv_y = double(dh) / sh;
    const double scale_x = 1.0 / inv_x, scale_y = 1.0 / inv_y;
    const int isx = int(std::nearbyint(scale_x)), isy = int(std::nearbyint(scale_y));
    const bool fast = std::abs(scale_x - isx) < DBL_EPSILON && std::abs(scale_y - isy) < DBL_EPSILON;
    if (interpolation == 1 && fast && isx == 2 && isy == 2) interpolation = 3;
    if (interpolation == 3) {
        if (!(scale_x >= 1 && scale_y >= 1)) return false;
        if (fast) {
            p.kind = 2;
            p.ix = isx;
            p.iy = isy;
            p.fscale = 1.f / float(isx * isy);
            return true;
        }
        p.kind = 1;
        index_taps(area_taps(sw, dw, scale_x), dw, p.xfirst, p.xsi, p.xal);
        index_taps(area_taps(sh, dh, scale_y), dh, p.yfirst, p.ysi, p.yal);
        return true;
    }
    if (interpolation != 1) return false;
    p.kind = 3;
    p.lxmax = dw;
    for (int dx = 0; dx < dw; ++dx) {
        float fx = float((dx + 0.5) * scale_x - 0.5);
        int sx = int(std::floor(fx));
        fx -= float(sx);
        if (sx < 0) { fx = 0.f; sx = 0; }
        if (sx + 1 >= sw) {
            p.lxmax = std::min(p.lxmax, dx);
            if (sx >= sw - 1) { fx = 0.f; sx = sw - 1; }
        }
        p.lxofs.push_back(sx);
        p.lalpha.push_back(std::max(-32768, std::min(32767, rint_f((1.f - fx) * COEF_SCALE))));
        p.lalpha.push_back(std::max(-32768, std::min(32767, rint_f(fx * COEF_SCALE))));
    }
    for (int dy = 0; dy < dh; ++dy) {
        float fy = float((dy + 0.5) * scale_y - 0.5);
        const int sy = int(std::floor(fy));
        fy -= float(sy);
        p.lyofs.push_back(sy);
        p.lbeta.push_back(std::max(-32768, std::min(32767, rint_f((1.f - fy) * COEF_SCALE))));
        p.lbeta.push_back(std::max(-32768, std::min(32767, rint_f(fy * COEF_SCALE))));
    }
    return true;
}

// 16-bit rounding of a 2^16-scaled coefficient with saturation (ffmpeg's round + av_clip_int16)
int round_to_16(long long f) {
    int r = int((f + (1 << 15)) >> 16);
    if (r < -32768) r = -32768;
    if (r > 32767) r = 32767;
    return r;
}
Yuv yuv_coeffs() {
    const long long cy = (65536LL * 255) / 219;   // contrast = saturation = 1 << 16 leave the table entries unscaled
    Yuv k;
    k.y_coeff = round_to_16(cy * (1 << 13));
    k.vr = round_to_16(104597LL * (1 << 13));
    k.ub = round_to_16(132201LL * (1 << 13));
    k.ug = round_to_16(-25675LL * (1 << 13));
    k.vg = round_to_16(-53279LL * (1 << 13));
    k.y_off = round_to_16((16LL << 16) * (1 << 3));
    k.uv_off = 0x0400;
    return k;
}

// canvas geometry of a w x h frame (geometry.cpp:77-88): scale min(720/h, 1280/w), centred, mode 0 copy /
// 1 shrink (area) / 2 enlarge (linear)
struct CanvasGeo {
    int new_w, new_h, left, top, mode;
};
bool canvas_geo(int w, int h, CanvasGeo& g) {
    if (w <= 0 || h <= 0) return false;
    const double scale = std::min(720.0 / h, 1280.0 / w);
    g.new_h = int(std::max(1L, py_round(h * scale)));
    g.new_w = int(std::max(1L, py_round(w * scale)));
    if (g.new_w > 1280 || g.new_h > 720) return false;
    g.left = (1280 - g.new_w) / 2;
    g.top = (720 - g.new_h) / 2;
    g.mode = (g.new_h == h && g.new_w == w) ? 0 : (scale < 1 ? 1 : 2);
    return true;
}

// Plans uploaded once per geometry; the device plan table and scratch grow as needed.  One call at a time.
class CropEngine {
public:
    static CropEngine& get() {
        static CropEngine e;
        return e;
    }
    void run(const CropJob* jobs, int n, uint8_t* out, hipStream_t s, bool i420) {
        // every argument is checked before the device is touched
        std::vector<CanvasGeo> geo(static_cast<size_t>(n));
        for (int i = 0; i < n; ++i) {
            const CropJob& j = jobs[i];
            if (!j.frame || j.width <= 0 || j.height <= 0 || j.stride < (i420 ? 1LL : 3LL) * j.width ||
                (i420 && (!j.u || !j.v || j.u_stride < (j.width + 1) / 2 || j.v_stride < (j.width + 1) / 2)))
                throw std::runtime_error("crops: bad frame " + std::to_string(i));
            if (j.x < 0 || j.y < 0 || j.w <= 0 || j.h <= 0 || j.x + j.w > CROP_W || j.y + j.h > CROP_H)
                throw std::runtime_error("crops: rect out of the 320x180 letterbox at crop " + std::to_string(i));
            if (4 * j.w < CROP_W || 4 * j.h < CROP_H)
                throw std::runtime_error("crops: rect smaller than 80x45 (no INTER_AREA shrink) at crop " +
                                         std::to_string(i));
            if (!canvas_geo(j.width, j.height, geo[size_t(i)])) throw std::runtime_error("crops: frame size");
        }
        std::lock_guard<std::mutex> lk(mu_);
        int dev = 0;
        CROP_CHECK(hipGetDevice(&dev));
        if (device_ >= 0 && dev != device_) throw std::runtime_error("crops: one device per process");
        device_ = dev;
        std::vector<JobDev> jd(static_cast<size_t>(n));
        long long scratch = 0;
        int max_ph = 0;
        for (int i = 0; i < n; ++i) {
            const CropJob& j = jobs[i];
            const CanvasGeo& g = geo[size_t(i)];
            JobDev& d = jd[size_t(i)];
            d.frame = j.frame;
            d.stride = j.stride;
            d.u = j.u; d.v = j.v; d.u_stride = j.u_stride; d.v_stride = j.v_stride;
            d.canvas_plan = plan_index(0, j.width, j.height, g.new_w, g.new_h, g.mode == 2 ? 1 : 3);
            d.crop_plan = plan_index(1, 4 * j.w, 4 * j.h, CROP_W, CROP_H, 3);
            d.px0 = 4 * j.x; d.py0 = 4 * j.y; d.pw = 4 * j.w; d.ph = 4 * j.h;
            d.left = g.left; d.top = g.top; d.new_w = g.new_w; d.new_h = g.new_h;
            d.patch_off = scratch;
            scratch += (3LL * d.pw * d.ph + 255) / 256 * 256;
            max_ph = std::max(max_ph, d.ph);
        }
        sync_plans();
        grow(scratch_, scratch_bytes_, size_t(scratch));
        grow(jobs_dev_, jobs_bytes_, jd.size() * sizeof(JobDev));
        CROP_CHECK(hipMemcpyAsync(jobs_dev_, jd.data(), jd.size() * sizeof(JobDev), hipMemcpyHostToDevice, s));
        const JobDev* jdev = static_cast<const JobDev*>(jobs_dev_);
        static const Yuv yuv = yuv_coeffs();
        if (i420)
            hipLaunchKernelGGL(crop_patch_kernel<true>, dim3(max_ph, n), dim3(256), 0, s, jdev,
                               static_cast<const PlanDev*>(plans_dev_), static_cast<uint8_t*>(scratch_), yuv);
        else
            hipLaunchKernelGGL(crop_patch_kernel<false>, dim3(max_ph, n), dim3(256), 0, s, jdev,
                               static_cast<const PlanDev*>(plans_dev_), static_cast<uint8_t*>(scratch_), yuv);
        CROP_CHECK(hipGetLastError());
        hipLaunchKernelGGL(crop_resize_kernel, dim3(CROP_H, n), dim3(256), 0, s, jdev,
                           static_cast<const PlanDev*>(plans_dev_), static_cast<const uint8_t*>(scratch_), out);
        CROP_CHECK(hipGetLastError());
        CROP_CHECK(hipStreamSynchronize(s));   // the job table and scratch are reused by the next call
    }

private:
    std::mutex mu_;
    int device_ = -1;
    std::map<std::vector<int>, int> index_;   // (role, sw, sh, dw, dh, interpolation) -> plan
    std::vector<PlanDev> plans_;
    std::vector<void*> tables_;               // device copies of the plan tables
    bool plans_dirty_ = false;
    void *plans_dev_ = nullptr, *scratch_ = nullptr, *jobs_dev_ = nullptr;
    size_t plans_bytes_ = 0, scratch_bytes_ = 0, jobs_bytes_ = 0;

    static void grow(void*& p, size_t& have, size_t need) {
        if (need <= have) return;
        if (p) CROP_CHECK(hipFree(p));
        p = nullptr;
        have = 0;
        CROP_CHECK(hipMalloc(&p, need));
        have = need;
    }
    template <class V> const typename V::value_type* upload(const V& v) {
        if (v.empty()) return nullptr;
        void* d = nullptr;
        CROP_CHECK(hipMalloc(&d, v.size() * sizeof(typename V::value_type)));
        tables_.push_back(d);
        CROP_CHECK(hipMemcpy(d, v.data(), v.size() * sizeof(typename V::value_type), hipMemcpyHostToDevice));
        return static_cast<const typename V::value_type*>(d);
    }
    int plan_index(int role, int sw, int sh, int dw, int dh, int interp) {
        const std::vector<int> key{role, sw, sh, dw, dh, interp};
        auto it = index_.find(key);
        if (it != index_.end()) return it->second;
        PlanHost h;
        if (!make_plan(sw, sh, dw, dh, interp, h)) throw std::runtime_error("crops: no resize plan for this geometry");
        PlanDev d;
        d.kind = h.kind; d.sw = h.sw; d.sh = h.sh; d.dw = h.dw; d.dh = h.dh;
        d.ix = h.ix; d.iy = h.iy; d.fscale = h.fscale; d.lxmax = h.lxmax;
        d.xfirst = upload(h.xfirst); d.xsi = upload(h.xsi); d.xal = upload(h.xal);
        d.yfirst = upload(h.yfirst); d.ysi = upload(h.ysi); d.yal = upload(h.yal);
        d.lxofs = upload(h.lxofs); d.lalpha = upload(h.lalpha); d.lyofs = upload(h.lyofs); d.lbeta = upload(h.lbeta);
        plans_.push_back(d);
        plans_dirty_ = true;
        return index_[key] = int(plans_.size() - 1);
    }
    void sync_plans() {
        if (!plans_dirty_) return;
        grow(plans_dev_, plans_bytes_, plans_.size() * sizeof(PlanDev));
        CROP_CHECK(hipMemcpy(plans_dev_, plans_.data(), plans_.size() * sizeof(PlanDev), hipMemcpyHostToDevice));
        plans_dirty_ = false;
    }
};

}  // namespace

void native_crops(const CropJob* jobs, int n, uint8_t* out, bool i420, hipStream_t s) {
    if (n <= 0) return;
    if (!jobs || !out || n > 65535) throw std::runtime_error("crops: null buffer or more than 65535 crops");
    CropEngine::get().run(jobs, n, out, s, i420);
}

}  // namespace shv
