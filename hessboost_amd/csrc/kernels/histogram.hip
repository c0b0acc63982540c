// Gradient histograms in fixed point (the hot kernel of tree growth).
//
// Replaces CpuBackend::build (tree/hist/mod.rs:510-547): every bin of a node
// receives the integer sum of its rows' quantized (g, h). Integer sums are
// exact and order-free, so any launch shape, tile size or workgroup count
// gives the same bins; when the reference's own sums are exact
// (backend/exact_sum.rs:14-37) these equal its f64 bins bit for bit.
//
// Dense indexes read row-major local bins (u8 for <= 256 bins per feature):
// a workgroup takes a tile of one node's rows and a group of features,
// accumulates into an LDS sub-histogram with 64-bit integer atomics, and
// flushes the non-zero bins to the node's slot with 64-bit global atomics.
// Sparse (CSR) indexes add each stored entry straight to the slot.
#include "common.h"

namespace hbr {

__device__ __forceinline__ Seg resolve_node(const HistArgs &a, const HistNode &nd) {
    if (!nd.from_split) return nd.seg;
    const PartSplit sp = a.splits[nd.split];
    const PartOut po = a.part_out[nd.split];
    Seg s;
    s.buf = sp.seg.buf ^ 1u;
    s.pad = 0;
    if (po.built_left) {
        s.offset = sp.seg.offset;
        s.len = po.left_len;
    } else {
        s.offset = sp.seg.offset + po.left_len;
        s.len = sp.seg.len - po.left_len;
    }
    return s;
}

template <int FG>
__device__ __forceinline__ void hist_dense8(const HistArgs &a) {
    __shared__ unsigned long long lds[FG * 256 * 2];
    const HistTile t = a.tiles[blockIdx.x];
    const HistNode nd = a.nodes[t.node];
    const Seg seg = resolve_node(a, nd);
    if (t.row0 >= seg.len) return;  // uniform across the workgroup
    const uint32_t end = min(t.row0 + a.tile_rows, seg.len);
    const uint32_t nf = t.nf;
    for (uint32_t i = threadIdx.x; i < nf * 512u; i += blockDim.x) lds[i] = 0ull;
    __syncthreads();
    const int eg = a.scale->exp_g, eh = a.scale->exp_h;
    const uint32_t *rows = a.rows[seg.buf];
    const uint32_t nw = (nf + 3) / 4;
    for (uint32_t j = t.row0 + threadIdx.x; j < end; j += blockDim.x) {
        const uint32_t r = nd.contiguous ? seg.offset + j : rows[seg.offset + j];
        const GPair p = a.gpair[r];
        const unsigned long long qg = (unsigned long long)quantize(p.g, eg);
        const unsigned long long qh = (unsigned long long)quantize(p.h, eh);
        const uint32_t *b = (const uint32_t *)(a.bins8 + (size_t)r * a.stride + t.f0);
        uint32_t words[(FG + 3) / 4];
#pragma unroll
        for (int w = 0; w < (FG + 3) / 4; w++) words[w] = (uint32_t)w < nw ? b[w] : 0u;
#pragma unroll
        for (int f = 0; f < FG; f++) {
            if ((uint32_t)f < nf) {
                const uint32_t bin = (words[f >> 2] >> ((f & 3) * 8)) & 0xffu;
                const uint32_t at = ((uint32_t)f * 256u + bin) * 2u;
                atomicAdd(&lds[at], qg);
                atomicAdd(&lds[at + 1], qh);
            }
        }
    }
    __syncthreads();
    QBin *dst = a.hist + (size_t)nd.slot * a.total_bins;
    const uint32_t *fo = a.feature_offset + t.f0;
    for (uint32_t i = threadIdx.x; i < nf * 256u; i += blockDim.x) {
        const uint32_t f = i >> 8, bin = i & 255u;
        const uint32_t lo = fo[f], nb = fo[f + 1] - lo;
        if (bin >= nb) continue;
        const unsigned long long g = lds[2 * i], h = lds[2 * i + 1];
        if ((g | h) == 0ull) continue;
        atomicAdd((unsigned long long *)&dst[lo + bin].g, g);
        atomicAdd((unsigned long long *)&dst[lo + bin].h, h);
    }
}

__device__ __forceinline__ void hist_csr(const HistArgs &a) {
    const HistTile t = a.tiles[blockIdx.x];
    const HistNode nd = a.nodes[t.node];
    const Seg seg = resolve_node(a, nd);
    if (t.row0 >= seg.len) return;
    const uint32_t end = min(t.row0 + a.tile_rows, seg.len);
    const int eg = a.scale->exp_g, eh = a.scale->exp_h;
    const uint32_t *rows = a.rows[seg.buf];
    QBin *dst = a.hist + (size_t)nd.slot * a.total_bins;
    for (uint32_t j = t.row0 + threadIdx.x; j < end; j += blockDim.x) {
        const uint32_t r = nd.contiguous ? seg.offset + j : rows[seg.offset + j];
        const GPair p = a.gpair[r];
        const unsigned long long qg = (unsigned long long)quantize(p.g, eg);
        const unsigned long long qh = (unsigned long long)quantize(p.h, eh);
        for (uint64_t e = a.row_ptr[r]; e < a.row_ptr[r + 1]; e++) {
            const uint32_t gb = a.gbins[e];
            atomicAdd((unsigned long long *)&dst[gb].g, qg);
            atomicAdd((unsigned long long *)&dst[gb].h, qh);
        }
    }
}

}  // namespace hbr

using namespace hbr;

extern "C" __global__ __launch_bounds__(512) void hbr_hist_dense8_fg8(HistArgs a) { hist_dense8<8>(a); }
extern "C" __global__ __launch_bounds__(512) void hbr_hist_dense8_fg16(HistArgs a) { hist_dense8<16>(a); }
extern "C" __global__ __launch_bounds__(512) void hbr_hist_dense8_fg32(HistArgs a) { hist_dense8<32>(a); }
extern "C" __global__ __launch_bounds__(512) void hbr_hist_csr(HistArgs a) { hist_csr(a); }

// sibling = parent - built (exact in integers), in the parent's slot.
extern "C" __global__ __launch_bounds__(256) void hbr_subtract(SubArgs a) {
    const uint32_t s = blockIdx.y;
    if (s >= a.n_splits) return;
    const PartSplit sp = a.splits[s];
    QBin *parent = a.hist + (size_t)sp.parent_slot * a.total_bins;
    const QBin *built = a.hist + (size_t)sp.fresh_slot * a.total_bins;
    for (uint32_t b = blockIdx.x * blockDim.x + threadIdx.x; b < a.total_bins; b += gridDim.x * blockDim.x) {
        QBin p = parent[b];
        const QBin c = built[b];
        p.g -= c.g;
        p.h -= c.h;
        parent[b] = p;
    }
}

extern "C" __global__ __launch_bounds__(256) void hbr_zero_slots(ZeroArgs a) {
    const uint32_t s = blockIdx.y;
    if (s >= a.n_slots) return;
    QBin *h = a.hist + (size_t)a.slots[s] * a.total_bins;
    for (uint32_t b = blockIdx.x * blockDim.x + threadIdx.x; b < a.total_bins; b += gridDim.x * blockDim.x)
        h[b] = QBin{0, 0};
}
