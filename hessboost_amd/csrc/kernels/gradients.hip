// Gradient kernels: squared error and the logistic loss, with the host's
// exact f32 operations, plus the per-tree quantization scale.
//
// Squared error restates objective/regression.rs:42-58: w scaled by
// scale_pos_weight for a label of exactly 1, g = (p - y) w, h = w.
//
// The logistic loss restates the reference's AVX2/FMA vector kernel
// (simd/x86_64.rs:22-160) one lane per row: a row belongs to the 8-row
// vector [8k, 8k + 8) and takes the polynomial path only when every margin
// of that vector is finite with magnitude <= 80 and the vector lies below
// vec_rows (simd/mod.rs:57-66). Each intrinsic becomes the same single IEEE
// f32 operation: _mm256_fmadd_ps/_fnmadd_ps are fmaf, _mm256_cvtps_epi32 is
// round-to-nearest-even, divisions are correctly rounded. Rows outside that
// path take the scalar sigmoid, 1 / (expf(min(-x, 88.7)) + 1)
// (simd/mod.rs:425-427, simd/scalar.rs:8-29), with the host libm's expf
// restated bit for bit.
#include "common.h"
#include "libm_expf.h"

namespace hbr {

// Exponential of x in [-80, 0] as simd/x86_64.rs:22-51 computes it.
__device__ __forceinline__ float exp_vector(float x) {
    float t = x * 1.44269504088896341f;
    int k = (int)__builtin_rintf(t);
    float kf = (float)k;
    float r = __builtin_fmaf(-kf, 0.6933594f, x);
    r = __builtin_fmaf(kf, 2.1219444e-4f, r);
    float r2 = r * r;
    float r4 = r2 * r2;
    float p0 = 1.0f + r;
    float p1 = __builtin_fmaf(1.0f / 6.0f, r, 0.5f);
    float p2 = __builtin_fmaf(1.0f / 120.0f, r, 1.0f / 24.0f);
    float p3 = __builtin_fmaf(1.0f / 5040.0f, r, 1.0f / 720.0f);
    float lo = __builtin_fmaf(p1, r2, p0);
    float hi = __builtin_fmaf(p3, r2, p2);
    float poly = __builtin_fmaf(hi, r4, lo);
    uint32_t bits = (uint32_t)(k + 127) << 23;
    return poly * __uint_as_float(bits);
}

// Workgroup-wide fold of the magnitude maxima and the non-finite count,
// then one atomic per workgroup (non-negative f32 bits order as integers).
__device__ __forceinline__ void fold_block(QScale *s, uint32_t mg, uint32_t mh, uint32_t bad) {
    __shared__ uint32_t red[3][1024 / kWave];  // workgroups of up to 1024 threads
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        mg = max(mg, (uint32_t)__shfl_xor((int)mg, d, kWave));
        mh = max(mh, (uint32_t)__shfl_xor((int)mh, d, kWave));
        bad += (uint32_t)__shfl_xor((int)bad, d, kWave);
    }
    const uint32_t wave = threadIdx.x / kWave;
    if (lane_id() == 0) {
        red[0][wave] = mg;
        red[1][wave] = mh;
        red[2][wave] = bad;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < blockDim.x / kWave; w++) {
            mg = max(mg, red[0][w]);
            mh = max(mh, red[1][w]);
            bad += red[2][w];
        }
        if (mg) atomicMax(&s->max_g_bits, mg);
        if (mh) atomicMax(&s->max_h_bits, mh);
        if (bad) atomicAdd(&s->nonfinite, bad);
    }
}

}  // namespace hbr

using namespace hbr;

namespace hbr {

// The scalar sigmoid's pair (simd/mod.rs:425-427, simd/scalar.rs:8-29):
// p = 1 / (expf(min(-m, 88.7)) + 1), w scaled for a label of exactly 1.
__device__ __forceinline__ GPair logistic_scalar_pair(const GradArgs &a, float m, float y, float w, float *p_out) {
    const float p = 1.0f / (hbr_expf_libm(__builtin_fminf(-m, 88.7f), a.exp_table) + 1.0f);
    const float ww = w * (y == 1.0f ? a.scale_pos_weight : 1.0f);
    *p_out = p;
    return GPair{(p - y) * ww, __builtin_fmaxf(p * (1.0f - p), a.min_hess) * ww};
}

// The word a row carries for its logistic pair (GradArgs::pair_rows).
__device__ __forceinline__ uint32_t pair_word(float p, float y) {
    return __float_as_uint(p) | (y == 1.0f ? 0x80000000u : 0u);
}

// The vector path's pair (simd/x86_64.rs:53-160, one lane): p from the
// polynomial exponential of -|m|, w scaled for a label of exactly 1.
__device__ __forceinline__ GPair logistic_vector_pair(const GradArgs &a, float m, float y, float w, float *p_out) {
    const float e = exp_vector(0.0f - __builtin_fabsf(m));
    const float den = 1.0f + e;
    const float pos = 1.0f / den;
    const float neg = e / den;
    const float p = m >= 0.0f ? pos : neg;
    const float ww = w * (y == 1.0f ? a.scale_pos_weight : 1.0f);
    const float q = p * (1.0f - p);
    *p_out = p;
    return GPair{(p - y) * ww, (q > a.min_hess ? q : a.min_hess) * ww};
}

// A row of the vector range whose margin fails the vector test marks its
// original 8-row vector for hbr_regroup (rows held reordered).
__device__ __forceinline__ void mark_group(const GradArgs &a, uint32_t orig) {
    const uint32_t g = orig >> 3;
    if (atomicExch(&a.group_stamp[g], a.stamp) != a.stamp) a.bad_groups[1u + atomicAdd(&a.bad_groups[0], 1u)] = g;
}

// Row i's gradient pair from margin m, label y and weight w (all lanes of
// the wave call it together: the logistic vector test is a ballot over
// 8-row groups). orig: the row's original index (i unless the rows are
// held reordered, GradArgs::perm; the test is then the row's own, and
// hbr_regroup finishes it). kDefer: a row outside the vector path is
// listed for hbr_finish_scale instead (keeping the f64 expf out of a hot
// loop). *word: the row's pair word (pair_word) when its logistic pair is
// computed here (left alone for a deferred row). *pair (when given): the
// row's pair, set for an active row whose pair is computed here.
template <bool kDefer>
__device__ __forceinline__ void row_gradient_yw(const GradArgs &a, uint32_t i, uint32_t orig, bool active, float m,
                                                float y, float w, uint32_t &mg, uint32_t &mh, uint32_t &bad,
                                                uint32_t *word, GPair *pair = nullptr) {
    {
        float g = 0.0f, h = 0.0f;
        if (a.loss == kSquaredError) {
            if (y == 1.0f) w *= a.scale_pos_weight;
            g = (m - y) * w;
            h = w;
        } else {
            bool ok = active && __builtin_fabsf(m) <= a.max_input;
            bool vector;
            if (a.perm) {
                const bool in_range = orig < a.vec_rows;
                vector = ok && in_range;
                if (active && !ok && in_range) mark_group(a, orig);
            } else {
                uint64_t ballot = __ballot(ok || !active);
                uint64_t group = 0xffull << (lane_id() & ~7u);
                vector = active && i < a.vec_rows && (ballot & group) == group;
            }
            if (vector) {
                float p;
                const GPair q = logistic_vector_pair(a, m, y, w, &p);
                g = q.g;
                h = q.h;
                *word = pair_word(p, y);
            } else if (active) {
                if (kDefer) {
                    a.scalar_list[atomicAdd(&a.scale->scalar_rows, 1u)] = i;
                    return;
                }
                float p;
                const GPair q = logistic_scalar_pair(a, m, y, w, &p);
                g = q.g;
                h = q.h;
                *word = pair_word(p, y);
            }
        }
        if (active) {
            if (a.gpair) a.gpair[i] = GPair{g, h};  // null: the rows carry the pairs alone
            if (pair) *pair = GPair{g, h};
            mg = max(mg, __float_as_uint(g) & 0x7fffffffu);
            mh = max(mh, __float_as_uint(h) & 0x7fffffffu);
            bad += (!__builtin_isfinite(g) || !__builtin_isfinite(h)) ? 1u : 0u;
        }
    }
}

__device__ __forceinline__ void row_gradient(const GradArgs &a, uint32_t i, bool active, float m, uint32_t &mg,
                                             uint32_t &mh, uint32_t &bad) {
    const float y = active ? a.labels[i] : 0.0f;
    const float w = (active && a.weights) ? a.weights[i] : 1.0f;
    uint32_t word = 0;
    row_gradient_yw<false>(a, i, i, active, m, y, w, mg, mh, bad, &word);
    if (a.pair_rows && active)  // uniform flag; one word in the row's padding
        *reinterpret_cast<uint32_t *>(a.pair_rows + (size_t)i * a.pair_stride + a.pair_byte) = word;
}

}  // namespace hbr

// Grid-stride over rows; the stride is a multiple of 64, so every wave
// covers 64 consecutive rows and its lanes form whole 8-row vectors.
extern "C" __global__ __launch_bounds__(256) void hbr_gradients(GradArgs a) {
    uint32_t mg = 0, mh = 0, bad = 0;
    const uint32_t stride = gridDim.x * blockDim.x;
    const uint32_t end = (a.n + kWave - 1) / kWave * kWave;  // whole waves stay in the loop
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < end; i += stride) {
        const bool active = i < a.n;
        row_gradient(a, i, active, active ? a.margins[i] : 0.0f, mg, mh, bad);
    }
    fold_block(a.scale, mg, mh, bad);
}

// The exact domain's grains (backend/exact_sum.rs:244-254): for every
// finite nonzero g and h, the exponent of its lowest set bit; the smallest
// over the rows lands in scale->pad[0] (g) and pad[1] (h) as 1024 - (grain
// + 150), folded by maximum (0: every value zero; the memset leaves 0).
__device__ __forceinline__ uint32_t grain_fold_code(float v) {
    const uint32_t bits = __float_as_uint(v);
    const uint32_t biased = (bits >> 23) & 0xffu, mant = bits & 0x7fffffu;
    if (biased == 0xffu || (biased == 0u && mant == 0u)) return 0u;  // non-finite (counted elsewhere) or zero
    const uint32_t sig = biased == 0u ? mant : (mant | 0x800000u);
    const int32_t grain = (biased == 0u ? -149 : (int32_t)biased - 150) + (int32_t)__builtin_ctz(sig);
    return (uint32_t)(1024 - (grain + 150));
}

extern "C" __global__ __launch_bounds__(256) void hbr_grain_fold(GradArgs a) {
    uint32_t cg = 0, ch = 0;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += gridDim.x * blockDim.x) {
        const GPair p = a.gpair[i];
        cg = max(cg, grain_fold_code(p.g));
        ch = max(ch, grain_fold_code(p.h));
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        cg = max(cg, (uint32_t)__shfl_xor((int)cg, d, kWave));
        ch = max(ch, (uint32_t)__shfl_xor((int)ch, d, kWave));
    }
    if (lane_id() == 0) {
        if (cg) atomicMax(&a.scale->pad[0], cg);
        if (ch) atomicMax(&a.scale->pad[1], ch);
    }
}

extern "C" __global__ __launch_bounds__(256) void hbr_iota(IotaArgs a) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < a.n) a.rows[i] = a.first + i;
}

// Root statistics: the exact integer sums of the quantized pairs of a
// segment (order-free, so any launch shape gives the same totals).
extern "C" __global__ __launch_bounds__(256) void hbr_total(TotalArgs a) {
    const QScale *scale = a.scale + blockIdx.y;
    const GPair *gpair = a.gpair + blockIdx.y * a.tree_pairs;
    QBin *out = a.out + blockIdx.y;
    const int eg = scale->exp_g, eh = scale->exp_h;
    int64_t sg = 0, sh = 0;
    // eight rows a thread at a time, their loads issued together
    constexpr uint32_t kAhead = 8;
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t j0 = blockIdx.x * blockDim.x + threadIdx.x; j0 < a.n; j0 += kAhead * stride) {
        GPair p[kAhead];
#pragma unroll
        for (uint32_t k = 0; k < kAhead; k++) {
            const uint32_t j = j0 + k * stride;
            p[k] = GPair{0.0f, 0.0f};
            if (j < a.n) p[k] = gpair[a.rows ? a.rows[j] : a.first + j];
        }
#pragma unroll
        for (uint32_t k = 0; k < kAhead; k++) {
            sg += quantize(p[k].g, eg);
            sh += quantize(p[k].h, eh);
        }
    }
    __shared__ int64_t red[2][256 / kWave];
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        sg += __shfl_xor(sg, d, kWave);
        sh += __shfl_xor(sh, d, kWave);
    }
    if (lane_id() == 0) {
        red[0][threadIdx.x / kWave] = sg;
        red[1][threadIdx.x / kWave] = sh;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < blockDim.x / kWave; w++) {
            sg += red[0][w];
            sh += red[1][w];
        }
        atomicAdd((unsigned long long *)&out->g, (unsigned long long)sg);
        atomicAdd((unsigned long long *)&out->h, (unsigned long long)sh);
    }
}

// exp = e + ceil(log2 n) - 62 with M = m 2^e (m in [0.5, 1)) the maximum
// magnitude, 0 for a zero or non-finite maximum: the host's exponent rule.
__device__ __forceinline__ int32_t exponent_for(uint32_t bits, uint64_t rows) {
    if (bits == 0 || bits >= 0x7f800000u) return 0;
    int e = 0;
    (void)__builtin_frexpf(__uint_as_float(bits), &e);
    const int log_n = rows > 1 ? 64 - __builtin_clzll(rows - 1) : 0;
    return e + log_n - 62;
}

// One workgroup: the listed rows' pairs and their maxima, merged into the
// scale (read before anything here writes it), then the exponents.
extern "C" __global__ __launch_bounds__(256) void hbr_finish_scale(FinishArgs a) {
    if (blockIdx.x != 0) return;
    const QScale start = *a.scale;
    const uint32_t listed = a.grad.scalar_list ? start.scalar_rows : 0u;
    uint32_t mg = 0, mh = 0, bad = 0;
    for (uint32_t j = threadIdx.x; j < listed; j += blockDim.x) {
        const uint32_t r = a.grad.scalar_list[j];
        const float w = a.grad.weights ? a.grad.weights[r] : 1.0f;
        const float y = a.grad.labels[r];
        float pr;
        const GPair p = logistic_scalar_pair(a.grad, a.grad.margins[r], y, w, &pr);
        a.grad.gpair[r] = p;
        if (a.grad.pair_rows)
            *reinterpret_cast<uint32_t *>(a.grad.pair_rows + (size_t)r * a.grad.pair_stride + a.grad.pair_byte) =
                pair_word(pr, y);
        mg = max(mg, __float_as_uint(p.g) & 0x7fffffffu);
        mh = max(mh, __float_as_uint(p.h) & 0x7fffffffu);
        bad += (!__builtin_isfinite(p.g) || !__builtin_isfinite(p.h)) ? 1u : 0u;
    }
    __shared__ uint32_t red[3][256 / kWave];
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        mg = max(mg, (uint32_t)__shfl_xor((int)mg, d, kWave));
        mh = max(mh, (uint32_t)__shfl_xor((int)mh, d, kWave));
        bad += (uint32_t)__shfl_xor((int)bad, d, kWave);
    }
    if (lane_id() == 0) {
        red[0][threadIdx.x / kWave] = mg;
        red[1][threadIdx.x / kWave] = mh;
        red[2][threadIdx.x / kWave] = bad;
    }
    __syncthreads();
    if (threadIdx.x != 0) return;
    QScale q = start;
    for (uint32_t w = 0; w < blockDim.x / kWave; w++) {
        q.max_g_bits = max(q.max_g_bits, red[0][w]);
        q.max_h_bits = max(q.max_h_bits, red[1][w]);
        q.nonfinite += red[2][w];
    }
    q.deferred = listed;
    q.scalar_rows = 0;
    // bounds (when given) in place of the maxima, the larger should a maximum exceed its bound
    q.exp_g = exponent_for(max(q.max_g_bits, a.bound_g_bits), a.n_rows);
    q.exp_h = exponent_for(max(q.max_h_bits, a.bound_h_bits), a.n_rows);
    *a.scale = q;
}

extern "C" __global__ __launch_bounds__(64) void hbr_scale_rotate(RotateArgs a) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    *a.saved = *a.live;
    *a.live = QScale{};
}

extern "C" __global__ __launch_bounds__(64) void hbr_class_scales_finish(ScalesArgs a) {
    const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= a.k) return;
    QScale q = a.scales[c];
    q.exp_g = exponent_for(q.max_g_bits, a.n_rows);
    q.exp_h = exponent_for(q.max_h_bits, a.n_rows);
    q.scalar_rows = 0;
    a.scales[c] = q;
}

extern "C" __global__ __launch_bounds__(64) void hbr_scale_select(SelectArgs a) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    QScale q = *a.from;
    q.exp_g = exponent_for(q.max_g_bits, a.n_rows);
    q.exp_h = exponent_for(q.max_h_bits, a.n_rows);
    *a.to = q;
}

namespace hbr {

// Rust's saturating `label as usize` (simd/mod.rs:549): NaN and values below
// 1 give class 0, k stands for every index past the last class.
__device__ __forceinline__ uint32_t label_class(float y, uint32_t k) {
    if (!(y >= 1.0f)) return 0u;
    return y < (float)k ? (uint32_t)y : k;
}

}  // namespace hbr

// One thread per row, grid-stride over whole waves. The scalar row
// (simd/mod.rs:580-600): shift by max(f32::MIN_POSITIVE, margins), f64 sum
// of expf, p = expf(x - max) / (f32)sum, h = max(2p(1 - p)w, min_hess),
// g = (p - [class == label])w, with expf as the host libm computes it. The
// 2- and 4-class vector batches (simd/x86_64.rs:160-335): a batch of 8 / k
// consecutive rows is vectorised when each of its rows is free of NaN and
// max(f32::MIN_POSITIVE, row max) - row min <= 80 (the reference's lane
// permutes give every lane of a row these values); then e = the vector exp
// of x - max, the f32 row sum (e0 + e1, or (e0 + e1) + (e2 + e3)) and
// p = e * (1 / sum). Each class's magnitude maxima fold per wave, then per
// workgroup in LDS, then one atomic per class.
extern "C" __global__ __launch_bounds__(256) void hbr_softmax_grad(SoftmaxArgs a) {
    __shared__ uint64_t s_tab[32];
    __shared__ uint32_t s_fold[3][kSoftmaxMaxClasses];
    const uint32_t k = a.k;
    if (threadIdx.x < 32) s_tab[threadIdx.x] = a.exp_table[threadIdx.x];
    for (uint32_t c = threadIdx.x; c < k; c += blockDim.x) s_fold[0][c] = s_fold[1][c] = s_fold[2][c] = 0u;
    __syncthreads();
    const uint32_t per = k == 2 ? 4u : 2u;  // rows per vector batch (k = 2 or 4)
    const uint64_t group = (per == 4u ? 0xfull : 0x3ull) << (lane_id() & ~(per - 1u));
    const uint32_t stride = gridDim.x * blockDim.x;
    const uint32_t end = (a.n + kWave - 1) / kWave * kWave;  // whole waves stay in the loop
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < end; i += stride) {
        const bool active = i < a.n;
        const float *m = a.margins + (size_t)(active ? i : 0) * k;
        const float y = active ? a.labels[i] : 0.0f;
        const float w = (active && a.weights) ? a.weights[i] : 1.0f;
        const uint32_t label = label_class(y, k);
        // the vector batch test (a.batched is 0 unless k is 2 or 4)
        bool vec = false;
        float vmax = 0.0f, inv = 0.0f;
        if (a.batched) {
            const bool in_batch = i < a.batched;
            bool regular = false;
            if (in_batch) {
                float v[4];
#pragma unroll
                for (uint32_t c = 0; c < 4; c++) v[c] = c < k ? m[c] : v[0];
                bool nan = false;
                float hi = v[0], lo = v[0];
#pragma unroll
                for (uint32_t c = 0; c < 4; c++) {
                    nan |= __builtin_isnan(v[c]);
                    hi = __builtin_fmaxf(hi, v[c]);
                    lo = __builtin_fminf(lo, v[c]);
                }
                vmax = 0x1p-126f > hi ? 0x1p-126f : hi;
                regular = !nan && vmax - lo <= 80.0f;
                if (regular) {
                    float e[4];
#pragma unroll
                    for (uint32_t c = 0; c < 4; c++) e[c] = exp_vector(v[c] - vmax);
                    const float sum = k == 2 ? e[0] + e[1] : (e[0] + e[1]) + (e[2] + e[3]);
                    inv = 1.0f / sum;
                }
            }
            const uint64_t ok = __ballot(regular || !in_batch);
            vec = in_batch && (ok & group) == group;
        }
        float wmax = 0x1p-126f, ws = 1.0f;  // f32::MIN_POSITIVE
        if (active && !vec) {
            for (uint32_t c = 0; c < k; c++) wmax = __builtin_fmaxf(m[c], wmax);
            double sum = 0.0;
            for (uint32_t c = 0; c < k; c++) sum += (double)hbr_expf_libm(m[c] - wmax, s_tab);
            ws = (float)sum;
        }
        for (uint32_t c = 0; c < k; c++) {
            float g = 0.0f, h = 0.0f;
            if (active) {
                const float mc = m[c];
                if (vec) {
                    const float p = exp_vector(mc - vmax) * inv;
                    g = (p - (c == label ? 1.0f : 0.0f)) * w;
                    const float q = ((p * 2.0f) * (1.0f - p)) * w;
                    h = q > a.min_hess ? q : a.min_hess;
                } else {
                    const float p = hbr_expf_libm(mc - wmax, s_tab) / ws;
                    h = __builtin_fmaxf(2.0f * p * (1.0f - p) * w, a.min_hess);
                    g = (c == label ? p - 1.0f : p) * w;
                }
                a.gpair[(size_t)c * a.n + i] = GPair{g, h};
            }
            uint32_t mg = __float_as_uint(g) & 0x7fffffffu, mh = __float_as_uint(h) & 0x7fffffffu;
            const uint32_t bad =
                (uint32_t)__builtin_popcountll(__ballot(active && (!__builtin_isfinite(g) || !__builtin_isfinite(h))));
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) {
                mg = max(mg, (uint32_t)__shfl_xor((int)mg, d, kWave));
                mh = max(mh, (uint32_t)__shfl_xor((int)mh, d, kWave));
            }
            if (lane_id() == 0) {
                if (mg) atomicMax(&s_fold[0][c], mg);
                if (mh) atomicMax(&s_fold[1][c], mh);
                if (bad) atomicAdd(&s_fold[2][c], bad);
            }
        }
    }
    __syncthreads();
    for (uint32_t c = threadIdx.x; c < k; c += blockDim.x) {
        if (s_fold[0][c]) atomicMax(&a.scales[c].max_g_bits, s_fold[0][c]);
        if (s_fold[1][c]) atomicMax(&a.scales[c].max_h_bits, s_fold[1][c]);
        if (s_fold[2][c]) atomicAdd(&a.scales[c].nonfinite, s_fold[2][c]);
    }
}
