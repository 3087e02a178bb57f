// BLAKE3 in its default hash mode: the reference's file checksum (cli.py:34-39, written into the
// catalog whenever the blake3 package is installed, cli.py:48-53) and its tensor keys (repo3.py:529,
// :1029, siblings.py:216-240). Written from the published specification (O'Connor, Aumasson, Neves,
// Wilcox-O'Hearn, "BLAKE3: one function, fast everywhere", 2020): the compression function, 1 KiB
// chunks of 64-byte blocks, a binary tree of chaining values whose left subtrees are complete, ROOT
// on the last compression.
//
// Device (spa_blake3): any number of byte regions of one device buffer in a few launches. Stage 0
// gives a 256-lane workgroup 256 consecutive chunks of one region (a lane per chunk, 128 bytes per
// load step); the workgroup pairs their chaining values level by level in LDS, an odd last node
// carried up, down to one node: that is the subtree the tree holds over those chunks, because the
// chunks start at a multiple of 256 of their region (every aligned run of 2^k chunks is a complete
// subtree; a shorter run at a region's end reduces, with the same carry, to the node the whole tree
// holds there). Later stages do the same with 512 nodes per workgroup. The workgroup that holds a
// whole region's remaining nodes makes the last compression with ROOT and writes the digest.
//
// Host (spa_b3h_*): the incremental form (chunk chaining values pushed on a stack and merged while
// the chunk count is even, the last chunk held back for the root), the chunks of a large update
// hashed on threads, for files checked piece by piece as they are written.
#include <algorithm>
#include <string.h>
#include <thread>
#include <vector>

#include "../../include/seedpack_amd.h"
#include "launch.h"

namespace spa {
namespace b3 {

constexpr uint32_t IV0 = 0x6A09E667u, IV1 = 0xBB67AE85u, IV2 = 0x3C6EF372u, IV3 = 0xA54FF53Au,
                   IV4 = 0x510E527Fu, IV5 = 0x9B05688Cu, IV6 = 0x1F83D9ABu, IV7 = 0x5BE0CD19u;
constexpr uint32_t CHUNK_START = 1, CHUNK_END = 2, PARENT = 4, ROOT = 8;
constexpr int64_t CHUNK = 1024;
constexpr int LEAF_NODES = 256;     // chunks per stage-0 workgroup
constexpr int NODE_NODES = 512;     // chaining values per later-stage workgroup
constexpr int WG = 256;

// message word order of round r: the permutation (2 6 3 10 7 0 4 13 1 11 12 5 9 14 15 8) applied r times
struct Sched {
    uint8_t s[7][16];
    constexpr Sched() : s() {
        constexpr uint8_t P[16] = {2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8};
        for (int i = 0; i < 16; ++i) s[0][i] = (uint8_t)i;
        for (int r = 1; r < 7; ++r)
            for (int i = 0; i < 16; ++i) s[r][i] = s[r - 1][P[i]];
    }
};
constexpr Sched SCHED{};

__host__ __device__ __forceinline__ uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

#define B3_G(a, b, c, d, x, y)   \
    a = a + b + (x);             \
    d = rotr(d ^ a, 16);         \
    c = c + d;                   \
    b = rotr(b ^ c, 12);         \
    a = a + b + (y);             \
    d = rotr(d ^ a, 8);          \
    c = c + d;                   \
    b = rotr(b ^ c, 7)

// cv <- the chaining value of compressing block m (16 little-endian words) under cv
__host__ __device__ __forceinline__ void compress(uint32_t cv[8], const uint32_t m[16], uint64_t t, uint32_t len,
                                                  uint32_t flags) {
    uint32_t s0 = cv[0], s1 = cv[1], s2 = cv[2], s3 = cv[3], s4 = cv[4], s5 = cv[5], s6 = cv[6], s7 = cv[7];
    uint32_t s8 = IV0, s9 = IV1, s10 = IV2, s11 = IV3;
    uint32_t s12 = (uint32_t)t, s13 = (uint32_t)(t >> 32), s14 = len, s15 = flags;
#pragma unroll
    for (int r = 0; r < 7; ++r) {
        const uint8_t* q = SCHED.s[r];
        B3_G(s0, s4, s8, s12, m[q[0]], m[q[1]]);
        B3_G(s1, s5, s9, s13, m[q[2]], m[q[3]]);
        B3_G(s2, s6, s10, s14, m[q[4]], m[q[5]]);
        B3_G(s3, s7, s11, s15, m[q[6]], m[q[7]]);
        B3_G(s0, s5, s10, s15, m[q[8]], m[q[9]]);
        B3_G(s1, s6, s11, s12, m[q[10]], m[q[11]]);
        B3_G(s2, s7, s8, s13, m[q[12]], m[q[13]]);
        B3_G(s3, s4, s9, s14, m[q[14]], m[q[15]]);
    }
    cv[0] = s0 ^ s8; cv[1] = s1 ^ s9; cv[2] = s2 ^ s10; cv[3] = s3 ^ s11;
    cv[4] = s4 ^ s12; cv[5] = s5 ^ s13; cv[6] = s6 ^ s14; cv[7] = s7 ^ s15;
}

__host__ __device__ __forceinline__ void set_iv(uint32_t cv[8]) {
    cv[0] = IV0; cv[1] = IV1; cv[2] = IV2; cv[3] = IV3; cv[4] = IV4; cv[5] = IV5; cv[6] = IV6; cv[7] = IV7;
}

// out <- parent node of (l, r); out may alias neither
__host__ __device__ __forceinline__ void parent(const uint32_t l[8], const uint32_t r[8], bool root, uint32_t out[8]) {
    uint32_t m[16];
    for (int i = 0; i < 8; ++i) { m[i] = l[i]; m[8 + i] = r[i]; }
    set_iv(out);
    compress(out, m, 0, 64, PARENT | (root ? ROOT : 0));
}

// chaining value of a chunk of len (0..1024) bytes given by a byte reader
template <class Byte>
__host__ __device__ __forceinline__ void chunk_bytes(Byte byte, int64_t len, uint64_t counter, bool root, uint32_t cv[8]) {
    set_iv(cv);
    const int nb = len == 0 ? 1 : (int)((len + 63) / 64);
    for (int b = 0; b < nb; ++b) {
        uint32_t m[16];
        const int blen = (int)std::min<int64_t>(64, len - 64 * (int64_t)b);
        for (int w = 0; w < 16; ++w) {
            uint32_t v = 0;
            for (int k = 0; k < 4; ++k) {
                const int i = 4 * w + k;
                if (i < blen) v |= (uint32_t)byte(64 * (int64_t)b + i) << (8 * k);
            }
            m[w] = v;
        }
        uint32_t f = (b == 0 ? CHUNK_START : 0) | (b == nb - 1 ? CHUNK_END | (root ? ROOT : 0) : 0);
        compress(cv, m, counter, (uint32_t)blen, f);
    }
}

// ------------------------------------------------------------------ device

// one region at one stage: its workgroups start at blk0 (prefix over the stage's regions); n nodes
// (stage 0: bytes) at in (stage 0: byte offset into the data; later: node index into the input
// chaining values); its nodes out at out (node index), or its digest at region id `id` when this
// stage holds the whole region
struct StageRec {
    int64_t blk0, n, in, out;
    int32_t id, finish;
    int64_t pad;
};
static_assert(sizeof(StageRec) == 48, "StageRec layout");

__device__ __forceinline__ int find_rec(const StageRec* recs, int nrec, int64_t blk) {
    int lo = 0, hi = nrec - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (recs[mid].blk0 <= blk) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// the workgroup's m nodes in LDS reduced to node 0 (ROOT on the last parent when `finish`)
__device__ __forceinline__ void reduce_lds(uint32_t (*cvs)[9], int m, bool finish) {
    const int lane = threadIdx.x;
    while (m > 1) {
        const int half = (m + 1) >> 1;
        uint32_t v[8];
        if (lane < half) {
            if (2 * lane + 1 < m) {
                uint32_t l[8], r[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) { l[i] = cvs[2 * lane][i]; r[i] = cvs[2 * lane + 1][i]; }
                parent(l, r, finish && m == 2, v);
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = cvs[2 * lane][i];
            }
        }
        __syncthreads();
        if (lane < half) {
#pragma unroll
            for (int i = 0; i < 8; ++i) cvs[lane][i] = v[i];
        }
        __syncthreads();
        m = half;
    }
}

__device__ __forceinline__ void store_node(const uint32_t (*cvs)[9], uint32_t* nodes, int64_t at, uint8_t* digests, int id,
                                           bool finish) {
    const int lane = threadIdx.x;
    if (lane < 8) {
        if (finish) reinterpret_cast<uint32_t*>(digests + 32 * (int64_t)id)[lane] = cvs[0][lane];
        else nodes[8 * at + lane] = cvs[0][lane];
    }
}

// stage 0: lane per chunk; full chunks read 128 bytes (8 x 16) per step when the region is 16-byte aligned
__global__ __launch_bounds__(WG) void k_b3_leaf(const uint8_t* __restrict__ data, const StageRec* __restrict__ recs, int nrec,
                                                uint32_t* __restrict__ out, uint8_t* __restrict__ digests) {
    __shared__ uint32_t cvs[LEAF_NODES][9];
    const StageRec rc = recs[find_rec(recs, nrec, blockIdx.x)];
    const int64_t j = blockIdx.x - rc.blk0;                   // the workgroup's block within the region
    const int64_t nchunks = rc.n == 0 ? 1 : (rc.n + CHUNK - 1) / CHUNK;
    const int m = (int)std::min<int64_t>(LEAF_NODES, nchunks - j * LEAF_NODES);
    const int lane = threadIdx.x;
    const bool finish = rc.finish != 0;
    if (lane < m) {
        const int64_t c = j * LEAF_NODES + lane;
        const int64_t len = std::min<int64_t>(CHUNK, rc.n - c * CHUNK);
        const uint8_t* p = data + rc.in + c * CHUNK;
        uint32_t cv[8];
        if (len == CHUNK && (reinterpret_cast<uintptr_t>(p) & 15) == 0) {
            set_iv(cv);
            const uint4* q = reinterpret_cast<const uint4*>(p);
            for (int b = 0; b < 16; b += 2) {
                uint4 v[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) v[k] = q[4 * b + k];
                uint32_t m0[16], m1[16];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    m0[4 * k] = v[k].x; m0[4 * k + 1] = v[k].y; m0[4 * k + 2] = v[k].z; m0[4 * k + 3] = v[k].w;
                    m1[4 * k] = v[4 + k].x; m1[4 * k + 1] = v[4 + k].y; m1[4 * k + 2] = v[4 + k].z; m1[4 * k + 3] = v[4 + k].w;
                }
                compress(cv, m0, (uint64_t)c, 64, b == 0 ? CHUNK_START : 0);
                compress(cv, m1, (uint64_t)c, 64, b == 14 ? CHUNK_END | (finish && nchunks == 1 ? ROOT : 0) : 0);
            }
        } else {
            chunk_bytes([p](int64_t i) { return p[i]; }, len, (uint64_t)c, finish && nchunks == 1, cv);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) cvs[lane][i] = cv[i];
    }
    __syncthreads();
    reduce_lds(cvs, m, finish);
    store_node(cvs, out, rc.out + j, digests, rc.id, finish);
}

// later stages: lane per pair of input nodes (the first level), then the LDS reduction
__global__ __launch_bounds__(WG) void k_b3_node(const uint32_t* __restrict__ in, const StageRec* __restrict__ recs, int nrec,
                                                uint32_t* __restrict__ out, uint8_t* __restrict__ digests) {
    __shared__ uint32_t cvs[WG][9];
    const StageRec rc = recs[find_rec(recs, nrec, blockIdx.x)];
    const int64_t j = blockIdx.x - rc.blk0;
    const int k = (int)std::min<int64_t>(NODE_NODES, rc.n - j * NODE_NODES);   // input nodes of this block
    const int m = (k + 1) >> 1;
    const int lane = threadIdx.x;
    const bool finish = rc.finish != 0;
    if (lane < m) {
        const int64_t a = rc.in + j * NODE_NODES + 2 * lane;
        uint32_t l[8], v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) l[i] = in[8 * a + i];
        if (2 * lane + 1 < k) {
            uint32_t r[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) r[i] = in[8 * (a + 1) + i];
            parent(l, r, finish && k == 2, v);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = l[i];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) cvs[lane][i] = v[i];
    }
    __syncthreads();
    reduce_lds(cvs, m, finish);
    store_node(cvs, out, rc.out + j, digests, rc.id, finish);
}

struct Plan {
    std::vector<StageRec> recs;      // all stages, back to back
    std::vector<int64_t> stage_at;   // first record of each stage (and the end)
    std::vector<int64_t> blocks;     // workgroups of each stage
    int64_t nodes_a = 0, nodes_b = 0;
};

// stage records of every stage for regions (offset, bytes): stage 0 over chunks, later over nodes
Plan plan_of(const uint64_t* regions, int nreg) {
    Plan p;
    std::vector<int64_t> n(nreg), in(nreg);
    std::vector<char> live(nreg, 1);
    for (int r = 0; r < nreg; ++r) { n[r] = (int64_t)regions[2 * r + 1]; in[r] = (int64_t)regions[2 * r]; }
    for (int stage = 0;; ++stage) {
        const int64_t cap = stage == 0 ? LEAF_NODES : NODE_NODES;
        p.stage_at.push_back((int64_t)p.recs.size());
        int64_t blk = 0, outn = 0;
        for (int r = 0; r < nreg; ++r) {
            if (!live[r]) continue;
            const int64_t nodes = stage == 0 ? (n[r] == 0 ? 1 : (n[r] + CHUNK - 1) / CHUNK) : n[r];
            const int64_t nb = (nodes + cap - 1) / cap;
            StageRec rc{};
            rc.blk0 = blk; rc.n = n[r]; rc.in = in[r]; rc.out = outn; rc.id = r; rc.finish = nb == 1;
            p.recs.push_back(rc);
            blk += nb;
            if (nb == 1) live[r] = 0;
            else { n[r] = nb; in[r] = outn; outn += nb; }
        }
        p.blocks.push_back(blk);
        if (stage % 2 == 0) p.nodes_a = std::max(p.nodes_a, outn);
        else p.nodes_b = std::max(p.nodes_b, outn);
        if (!outn) break;
    }
    p.stage_at.push_back((int64_t)p.recs.size());
    return p;
}

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

size_t work_of(const Plan& p, int nreg) {
    return align256(p.recs.size() * sizeof(StageRec)) + align256((size_t)p.nodes_a * 32) + align256((size_t)p.nodes_b * 32) +
           align256((size_t)nreg * 32);
}

// ------------------------------------------------------------------ host (incremental)

struct Host {
    uint32_t stack[64][8];
    int depth = 0;
    uint64_t chunks = 0;             // chunks pushed (all but the held one)
    uint8_t buf[CHUNK];
    int64_t buflen = 0;              // bytes of the held chunk
    bool held = false;               // buf holds a complete or partial chunk not yet pushed

    void push(const uint32_t cv[8]) {
        uint32_t c[8];
        memcpy(c, cv, 32);
        uint64_t total = ++chunks;
        while ((total & 1) == 0) {
            uint32_t p[8];
            parent(stack[--depth], c, false, p);
            memcpy(c, p, 32);
            total >>= 1;
        }
        memcpy(stack[depth++], c, 32);
    }
    void push_held() {
        uint32_t cv[8];
        const uint8_t* b = buf;
        chunk_bytes([b](int64_t i) { return b[i]; }, CHUNK, chunks, false, cv);
        push(cv);
        buflen = 0;
        held = false;
    }
};

void chunks_cv(const uint8_t* p, int64_t nchunks, uint64_t counter0, uint32_t (*out)[8], int threads) {
    auto work = [&](int64_t a, int64_t b) {
        for (int64_t c = a; c < b; ++c) {
            const uint8_t* q = p + c * CHUNK;
            chunk_bytes([q](int64_t i) { return q[i]; }, CHUNK, counter0 + (uint64_t)c, false, out[c]);
        }
    };
    threads = (int)std::max<int64_t>(1, std::min<int64_t>(threads, nchunks / 64));
    if (threads == 1) return work(0, nchunks);
    std::vector<std::thread> ts;
    for (int t = 0; t < threads; ++t) ts.emplace_back(work, nchunks * t / threads, nchunks * (t + 1) / threads);
    for (auto& t : ts) t.join();
}

}  // namespace b3
}  // namespace spa

using namespace spa;

extern "C" {

size_t spa_blake3_work_bytes(const uint64_t* regions, int nregions) {
    if (nregions <= 0 || !regions) return 0;
    return b3::work_of(b3::plan_of(regions, nregions), nregions);
}

int spa_blake3(const void* base, const uint64_t* regions, int nregions, void* work, size_t work_bytes, uint8_t* digests,
               void* stream) {
    if (nregions < 0) return fail(SPA_ERR_ARG, "spa_blake3: %d regions", nregions);
    if (!nregions) return SPA_OK;
    if (!regions || !digests || !work) return fail(SPA_ERR_ARG, "spa_blake3: null pointer");
    for (int r = 0; r < nregions; ++r)
        if (regions[2 * r + 1] && !base) return fail(SPA_ERR_ARG, "spa_blake3: null data with non-empty regions");
    const b3::Plan p = b3::plan_of(regions, nregions);
    const size_t need = b3::work_of(p, nregions);
    if (work_bytes < need) return fail(SPA_ERR_ARG, "spa_blake3: work of %zu bytes, %zu needed", work_bytes, need);
    hipStream_t st = (hipStream_t)stream;
    uint8_t* w = (uint8_t*)work;
    b3::StageRec* recs = (b3::StageRec*)w;
    uint32_t* na = (uint32_t*)(w + b3::align256(p.recs.size() * sizeof(b3::StageRec)));
    uint32_t* nb = (uint32_t*)((uint8_t*)na + b3::align256((size_t)p.nodes_a * 32));
    uint8_t* dg = (uint8_t*)nb + b3::align256((size_t)p.nodes_b * 32);
    SPA_HIP_TRY(hipMemcpyAsync(recs, p.recs.data(), p.recs.size() * sizeof(b3::StageRec), hipMemcpyHostToDevice, st));
    for (size_t s = 0; s + 1 < p.stage_at.size(); ++s) {
        const int64_t r0 = p.stage_at[s], nrec = p.stage_at[s + 1] - r0;
        if (!nrec) break;
        if (p.blocks[s] > 0x7fffffff) return fail(SPA_ERR_ARG, "spa_blake3: %lld workgroups", (long long)p.blocks[s]);
        uint32_t* out = s % 2 == 0 ? na : nb;
        if (s == 0)
            hipLaunchKernelGGL(b3::k_b3_leaf, dim3((unsigned)p.blocks[s]), dim3(b3::WG), 0, st, (const uint8_t*)base,
                               recs + r0, (int)nrec, out, dg);
        else
            hipLaunchKernelGGL(b3::k_b3_node, dim3((unsigned)p.blocks[s]), dim3(b3::WG), 0, st,
                               (const uint32_t*)(s % 2 == 0 ? nb : na), recs + r0, (int)nrec, out, dg);
        SPA_HIP_TRY(hipGetLastError());
    }
    SPA_HIP_TRY(hipMemcpyAsync(digests, dg, (size_t)nregions * 32, hipMemcpyDeviceToHost, st));
    SPA_HIP_TRY(hipStreamSynchronize(st));
    return SPA_OK;
}

int spa_b3h_new(void** h) {
    if (!h) return fail(SPA_ERR_ARG, "spa_b3h_new: null pointer");
    *h = new (std::nothrow) b3::Host();
    return *h ? SPA_OK : fail(SPA_ERR_ARG, "spa_b3h_new: out of memory");
}

int spa_b3h_update(void* hp, const void* data, size_t n, int threads) {
    if (!hp || (n && !data)) return fail(SPA_ERR_ARG, "spa_b3h_update: null pointer");
    b3::Host& h = *(b3::Host*)hp;
    const uint8_t* p = (const uint8_t*)data;
    while (n) {
        if (h.held && h.buflen == b3::CHUNK) h.push_held();         // more input: the held chunk is not the last
        if (h.buflen == 0 && n > (size_t)b3::CHUNK) {
            // whole chunks that more input follows, hashed in parallel, pushed in order
            const int64_t full = (int64_t)((n - 1) / b3::CHUNK);
            std::vector<uint32_t> cv((size_t)full * 8);
            b3::chunks_cv(p, full, h.chunks, reinterpret_cast<uint32_t(*)[8]>(cv.data()), threads);
            for (int64_t c = 0; c < full; ++c) h.push(&cv[(size_t)c * 8]);
            p += full * b3::CHUNK;
            n -= (size_t)full * b3::CHUNK;
            continue;
        }
        const size_t take = std::min<size_t>(n, (size_t)(b3::CHUNK - h.buflen));
        memcpy(h.buf + h.buflen, p, take);
        h.buflen += (int64_t)take;
        h.held = true;
        p += take;
        n -= take;
    }
    return SPA_OK;
}

int spa_b3h_final(void* hp, uint8_t* out32) {
    if (!hp || !out32) return fail(SPA_ERR_ARG, "spa_b3h_final: null pointer");
    const b3::Host& h = *(const b3::Host*)hp;
    uint32_t cv[8];
    const uint8_t* b = h.buf;
    const bool lone = h.chunks == 0;
    b3::chunk_bytes([b](int64_t i) { return b[i]; }, h.buflen, h.chunks, lone, cv);
    for (int d = h.depth - 1; d >= 0; --d) {
        uint32_t p[8];
        b3::parent(h.stack[d], cv, d == 0, p);
        memcpy(cv, p, 32);
    }
    for (int i = 0; i < 8; ++i)
        for (int k = 0; k < 4; ++k) out32[4 * i + k] = (uint8_t)(cv[i] >> (8 * k));
    return SPA_OK;
}

int spa_b3h_free(void* hp) {
    delete (b3::Host*)hp;
    return SPA_OK;
}

}  // extern "C"
