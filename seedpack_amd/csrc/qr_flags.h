// Block equality of a QR batch and the block-flag symbols, shared by the grid and non-grid coders.
//
// Most blocks of a file equal their prediction (each costs one flag symbol). Both the histogram and
// the encoder need, per block, whether it equals its prediction and whether the previous block of its
// segment did. k_qr_neq computes neq[b] for every block of the batch once, reading F and P as 16-byte
// words coalesced across the workgroup; k_qr_slots counts the flag symbols of all blocks with
// wave-aggregated atomics and lists the differing blocks, so that the modelling kernels run only on
// those (one lane or one wave each, all of them busy).
#pragma once

#include "launch.h"
#include "qr_model.h"

namespace spa {
namespace qr {
namespace {   // one copy per translation unit (the grid and non-grid coders both launch these)

// counts[key]++ for every active lane: one atomic per distinct key of the wave
__device__ __forceinline__ void hadd(uint32_t* counts, uint32_t key) {
    uint64_t pending = __ballot(1);
    const int lane = __lane_id();
    while (pending) {
        const int leader = __ffsll((unsigned long long)pending) - 1;
        const uint32_t k = __shfl(key, leader);
        const uint64_t same = __ballot(key == k) & pending;
        if (lane == leader) atomicAdd(&counts[k], (uint32_t)__popcll(same));
        pending &= ~same;
    }
}

// workspace: neq flags (one byte per block slot), the list length, the list (one u32 slot per block),
// per block its place in the list (u32), and for the non-grid encoder the symbols of the first `cap`
// listed blocks (maxsym u32 words and a u16 count each; cap = a sixteenth of the slots: blocks beyond
// it are modelled by the coder itself)
struct QrWork {
    uint8_t* neq;
    uint32_t* nlist;
    uint32_t* list;
    uint32_t* idx_of;
    uint16_t* nsym;
    uint32_t* syms;
    uint32_t* rcp;                     // (non-grid) the encoder's reciprocal per (table, symbol)
    uint32_t cap;
};
__host__ __device__ inline int64_t qr_sym_cap(int64_t slots) { return slots / 16 > 1024 ? slots / 16 : 1024; }
__host__ __device__ inline size_t qr_work_bytes(int64_t slots, int maxsym) {
    const size_t a = (size_t)((slots + 255) / 256 * 256), cap = (size_t)qr_sym_cap(slots);
    return a + 256 + (size_t)slots * 8 + (cap * 2 + 255) / 256 * 256 +
           (maxsym ? cap * (size_t)maxsym * 4 + (size_t)NTAB2 * 256 * 4 : 0);
}
__host__ __device__ inline QrWork qr_work(void* w, int64_t slots, int maxsym) {
    uint8_t* p = (uint8_t*)w;
    const size_t a = (size_t)((slots + 255) / 256 * 256), cap = (size_t)qr_sym_cap(slots);
    QrWork q;
    q.neq = p;
    q.nlist = (uint32_t*)(p + a);
    q.list = (uint32_t*)(p + a + 256);
    q.idx_of = q.list + slots;
    q.nsym = (uint16_t*)(q.idx_of + slots);
    q.syms = maxsym ? (uint32_t*)((uint8_t*)q.nsym + (cap * 2 + 255) / 256 * 256) : nullptr;
    q.rcp = maxsym ? q.syms + cap * (size_t)maxsym : nullptr;
    q.cap = maxsym ? (uint32_t)cap : 0;
    return q;
}

// neq[b] for the batch's blocks b < (last segment's b0 + nb): 256 blocks per workgroup. nlist (when
// given) is set to 0 for the k_qr_slots launch that follows on the stream.
__global__ __launch_bounds__(256) void k_qr_neq(const uint8_t* __restrict__ F, const uint8_t* __restrict__ P,
                                                const SG* __restrict__ sg, int nseg, int bs, uint8_t* __restrict__ neq,
                                                uint32_t* __restrict__ nlist) {
    __shared__ uint8_t fl[256];
    if (nlist && blockIdx.x == 0 && threadIdx.x == 0) *nlist = 0;
    const SG last = sg[nseg - 1];
    const int64_t nb = last.b0 + last.nb;
    const int64_t b0 = (int64_t)blockIdx.x * 256;
    if (b0 >= nb) return;
    const int nblk = (int)(nb - b0 < 256 ? nb - b0 : 256);
    fl[threadIdx.x] = 0;
    __syncthreads();
    const uint8_t* f = F + b0 * bs;
    const uint8_t* p = P + b0 * bs;
    const int nbytes = nblk * bs;
    int done = 0;
    if (((reinterpret_cast<uintptr_t>(f) | reinterpret_cast<uintptr_t>(p)) & 15) == 0) {
        const int nv = nbytes / 16;
        for (int i = threadIdx.x; i < nv; i += 256) {
            const uint4 a = reinterpret_cast<const uint4*>(f)[i], c = reinterpret_cast<const uint4*>(p)[i];
            const uint32_t x[4] = {a.x ^ c.x, a.y ^ c.y, a.z ^ c.z, a.w ^ c.w};
#pragma unroll
            for (int w = 0; w < 4; ++w)
                if (x[w])
                    for (int k = 0; k < 4; ++k)
                        if ((x[w] >> (8 * k)) & 0xffu) fl[(16 * i + 4 * w + k) / bs] = 1;
        }
        done = nv * 16;
    }
    for (int o = done + threadIdx.x; o < nbytes; o += 256)
        if (f[o] != p[o]) fl[o / bs] = 1;
    __syncthreads();
    if (threadIdx.x < nblk) neq[b0 + threadIdx.x] = fl[threadIdx.x];
}

// the flag symbol of every slot (segment s, block j) into counts; differing slots s * seg + j into list.
// The four flag counters (previous block equal, this block equal) are summed per lane over a
// grid-stride loop, then per wave and per workgroup: one global atomic per counter and workgroup
// (one per wave and block on a few addresses serialised in L2).
__global__ __launch_bounds__(256) void k_qr_slots(const SG* __restrict__ sg, int nseg, int seg,
                                                  const uint8_t* __restrict__ neq, uint32_t* __restrict__ counts,
                                                  uint32_t* __restrict__ list, uint32_t* __restrict__ nlist,
                                                  uint32_t* __restrict__ idx_of, uint32_t cap) {
    __shared__ uint32_t c4[4];
    if (threadIdx.x < 4) c4[threadIdx.x] = 0;
    __syncthreads();
    const int lane = __lane_id();
    uint32_t mine[4] = {0, 0, 0, 0};   // [prev * 2 + eq]
    const int64_t nslot = (int64_t)nseg * seg;
    for (int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; gid < nslot; gid += (int64_t)gridDim.x * blockDim.x) {
        const int64_t s = gid / seg;
        const int j = (int)(gid % seg);
        const SG g = sg[s];
        const bool valid = j < g.nb;
        int eq = 1;
        if (valid) {
            const int64_t b = g.b0 + j;
            eq = neq[b] ? 0 : 1;
            const int prev = j > 0 ? (neq[b - 1] ? 0 : 1) : 1;
            mine[prev * 2 + eq]++;
        }
        const uint64_t m = __ballot(valid && !eq);
        if (m) {
            const int leader = __ffsll((unsigned long long)m) - 1;
            uint32_t at = 0;
            if (lane == leader) at = atomicAdd(nlist, (uint32_t)__popcll(m));
            at = __shfl(at, leader);
            if (valid && !eq) {
                const uint32_t pos = at + (uint32_t)__popcll(m & ((1ull << lane) - 1));
                list[pos] = (uint32_t)gid;
                if (idx_of) idx_of[g.b0 + j] = pos < cap ? pos : 0xffffffffu;
            }
        }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        uint32_t v = mine[k];
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d);
        if (lane == 0 && v) atomicAdd(&c4[k], v);
    }
    __syncthreads();
    if (counts && threadIdx.x < 4 && c4[threadIdx.x])
        atomicAdd(&counts[(FLAG + (threadIdx.x >> 1)) * 256 + (threadIdx.x & 1)], c4[threadIdx.x]);
}

// F = P over the batch's blocks (b < last segment's b0 + nb) before a decode: the decoders then write
// only the blocks that differ, and the equal ones (most of a file) move as coalesced 16-byte words
// instead of one lane's byte loop per block
__global__ __launch_bounds__(256) void k_qr_prefill(uint8_t* __restrict__ F, const uint8_t* __restrict__ P,
                                                    const SG* __restrict__ sg, int nseg, int bs) {
    const SG last = sg[nseg - 1];
    const int64_t n = (last.b0 + last.nb) * bs;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t done = 0;
    if (((reinterpret_cast<uintptr_t>(F) | reinterpret_cast<uintptr_t>(P)) & 15) == 0) {
        const int64_t nv = n / 16;
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nv; i += stride)
            reinterpret_cast<uint4*>(F)[i] = reinterpret_cast<const uint4*>(P)[i];
        done = nv * 16;
    }
    for (int64_t i = done + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) F[i] = P[i];
}

inline int qr_prefill(void* F, const void* P, const void* sg, int nseg, int bs, hipStream_t st) {
    hipLaunchKernelGGL(k_qr_prefill, dim3(4096), dim3(256), 0, st, (uint8_t*)F, (const uint8_t*)P, (const SG*)sg, nseg, bs);
    SPA_HIP_TRY(hipGetLastError());
    return 0;
}

// neq flags, then the list of differing slots with (hist) the flag counts or (encode) each listed
// block's place in the list
inline int qr_flags(const void* F, const void* P, const void* sg, int nseg, int seg, int bs, const QrWork& w,
                    uint32_t* counts, bool places, hipStream_t st) {
    const int64_t slots = (int64_t)nseg * seg;
    const bool list = counts || places;
    hipLaunchKernelGGL(k_qr_neq, dim3((unsigned)((slots + 255) / 256)), dim3(256), 0, st, (const uint8_t*)F,
                       (const uint8_t*)P, (const SG*)sg, nseg, bs, w.neq, list ? w.nlist : nullptr);
    if (!list) {
        SPA_HIP_TRY(hipGetLastError());
        return 0;
    }
    const int64_t wgs = (slots + 255) / 256 < 8192 ? (slots + 255) / 256 : 8192;
    hipLaunchKernelGGL(k_qr_slots, dim3((unsigned)wgs), dim3(256), 0, st, (const SG*)sg, nseg, seg, (const uint8_t*)w.neq,
                       counts, w.list, w.nlist, places ? w.idx_of : nullptr, w.cap);
    SPA_HIP_TRY(hipGetLastError());
    return 0;
}

}  // namespace
}  // namespace qr
}  // namespace spa
