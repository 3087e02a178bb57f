// IQ lattice tables: codebook (grid), index map and neighbour lists of the six IQ grids, built on
// the host from the compact codebooks and uploaded once per device.
//
// For a point of the level lattice (index = sum of l_k << (b*k)) the map holds the grid point with
// exactly those levels, or -(offset+1) into the neighbour array, where the entry at offset is a count
// n followed by the n grid points nearest to it: all points in the `nwant` smallest distinct squared
// distances, in (distance, index) order. These are the tables llama.cpp's iq2xs_init_impl /
// iq3xs_init_impl build (ggml-quants.c:2854-3259, :3704-3903); the quantizers' results depend on their
// exact content and order. Distances are small integers, so each list is collected by a counting
// pass over distance buckets instead of a sort.
#include <hip/hip_runtime.h>

#include <mutex>
#include <thread>
#include <vector>

#include "../../include/seedpack_amd.h"
#include "iq_grids.h"
#include "iq_tables.h"
#include "launch.h"

namespace spa {
namespace {

struct Spec { const uint16_t* def; int size, npts, bits, kmap_size, nwant; };
// 0 IQ2_XXS, 1 IQ2_XS, 2 IQ1_S/IQ1_M, 3 IQ2_S, 4 IQ3_XXS, 5 IQ3_S
const Spec kSpecs[6] = {
    {IQ_GRID_0, 256, 8, 2, 43692, 2}, {IQ_GRID_1, 512, 8, 2, 43692, 2}, {IQ_GRID_2, 2048, 8, 2, 43692, 3},
    {IQ_GRID_3, 1024, 8, 2, 43692, 1}, {IQ_GRID_4, 256, 4, 3, 4096, 2}, {IQ_GRID_5, 512, 4, 3, 4096, 3},
};

struct Host {
    std::vector<uint8_t> grid;      // size * (8 or 4) bytes: coordinate values 2l+1
    std::vector<int32_t> map;
    std::vector<uint16_t> nb;
};

Host build(const Spec& s) {
    Host h;
    const int lmask = (1 << s.bits) - 1;
    h.grid.resize((size_t)s.size * s.npts);
    for (int k = 0; k < s.size; ++k)
        for (int i = 0; i < s.npts; ++i) h.grid[(size_t)k * s.npts + i] = (uint8_t)(2 * ((s.def[k] >> (s.bits * i)) & lmask) + 1);
    h.map.assign(s.kmap_size, -1);
    for (int k = 0; k < s.size; ++k) h.map[s.def[k]] = k;
    // neighbour lists of every index that is not a grid point, in index order
    std::vector<std::vector<uint16_t>> lists(s.kmap_size);
    const int nthreads = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    std::vector<std::thread> pool;
    for (int t = 0; t < nthreads; ++t)
        pool.emplace_back([&, t] {
            std::vector<int> d2(s.size);
            std::vector<int> cnt;
            for (int i = t; i < s.kmap_size; i += nthreads) {
                if (h.map[i] >= 0) continue;
                int pos[8];
                for (int k = 0; k < s.npts; ++k) pos[k] = 2 * ((i >> (s.bits * k)) & lmask) + 1;
                int dmax = 0;
                for (int j = 0; j < s.size; ++j) {
                    const uint8_t* pg = &h.grid[(size_t)j * s.npts];
                    int d = 0;
                    for (int k = 0; k < s.npts; ++k) d += (pg[k] - pos[k]) * (pg[k] - pos[k]);
                    d2[j] = d;
                    dmax = std::max(dmax, d);
                }
                cnt.assign(dmax + 1, 0);
                for (int j = 0; j < s.size; ++j) cnt[d2[j]]++;
                // the nwant smallest distances that occur, then every point at them, by (distance, index)
                std::vector<uint16_t>& out = lists[i];
                int have = 0;
                for (int d = 0; d <= dmax && have < s.nwant; ++d) {
                    if (!cnt[d]) continue;
                    ++have;
                    for (int j = 0; j < s.size; ++j)
                        if (d2[j] == d) out.push_back((uint16_t)j);
                }
            }
        });
    for (auto& th : pool) th.join();
    size_t total = 0;
    for (int i = 0; i < s.kmap_size; ++i)
        if (h.map[i] < 0) total += 1 + lists[i].size();
    h.nb.reserve(total);
    for (int i = 0; i < s.kmap_size; ++i) {
        if (h.map[i] >= 0) continue;
        h.map[i] = -(int32_t)(h.nb.size() + 1);
        h.nb.push_back((uint16_t)lists[i].size());
        h.nb.insert(h.nb.end(), lists[i].begin(), lists[i].end());
    }
    return h;
}

std::once_flag g_once[6];
Host g_host[6];

const Host& host_table(int idx) {
    std::call_once(g_once[idx], [idx] { g_host[idx] = build(kSpecs[idx]); });
    return g_host[idx];
}

constexpr int MAXDEV = 16;
std::mutex g_dev_mu;

// One table on one device: a single allocation holding grid, map and neighbour lists, filled by
// copies queued on the stream of the first call that needs it; `ready` is recorded after them and
// every later user's stream waits for it, so nothing on any stream reads the table before it is
// there, and no call blocks the host.
struct DevTable {
    IqDeviceTable t{};
    hipEvent_t ready = nullptr;
};
DevTable g_dev[MAXDEV][6];
// the device form of each table's map (list lengths packed beside their offsets), built once per
// process and kept: queued copies read it after the call that queued them has returned
std::once_flag g_dm_once[6];
std::vector<int32_t> g_dm[6];
int g_dm_err[6];

const std::vector<int32_t>& device_map(int idx) {
    std::call_once(g_dm_once[idx], [idx] {
        const Host& h = host_table(idx);
        std::vector<int32_t>& dm = g_dm[idx];
        dm.resize(h.map.size());
        for (size_t i = 0; i < h.map.size(); ++i) {
            const int32_t v = h.map[i];
            if (v >= 0) { dm[i] = v; continue; }
            const uint32_t off = (uint32_t)(-v - 1), len = h.nb[off];
            if (off >= (1u << 22) || len == 0 || len >= 512) { g_dm_err[idx] = 1; return; }
            dm[i] = -1 - (int32_t)((off << 9) | len);
        }
    });
    return g_dm[idx];
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

}  // namespace

int iq_table_index(int ggml_type) {
    switch (ggml_type) {
        case 16: return 0;
        case 17: return 1;
        case 19: case 29: return 2;
        case 22: return 3;
        case 18: return 4;
        case 21: return 5;
    }
    return -1;
}

int iq_device_table(int idx, IqDeviceTable* out, hipStream_t stream) {
    int dev = 0;
    SPA_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= MAXDEV || idx < 0 || idx > 5) return fail(SPA_ERR_ARG, "iq table %d on device %d", idx, dev);
    const Host& h = host_table(idx);
    const std::vector<int32_t>& dm = device_map(idx);
    if (g_dm_err[idx]) return fail(SPA_ERR_ARG, "iq table %d: a neighbour list does not fit the packed map", idx);
    std::lock_guard<std::mutex> lk(g_dev_mu);
    DevTable& d = g_dev[dev][idx];
    if (!d.t.grid) {
        const size_t og = 0, om = align256(h.grid.size()), on = om + align256(dm.size() * sizeof(int32_t));
        const size_t total = on + h.nb.size() * sizeof(uint16_t);
        uint8_t* base = nullptr;
        hipEvent_t ev = nullptr;
        hipError_t e = hipMalloc((void**)&base, total);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (e == hipSuccess) e = hipMemcpyAsync(base + og, h.grid.data(), h.grid.size(), hipMemcpyHostToDevice, stream);
        if (e == hipSuccess)
            e = hipMemcpyAsync(base + om, dm.data(), dm.size() * sizeof(int32_t), hipMemcpyHostToDevice, stream);
        if (e == hipSuccess)
            e = hipMemcpyAsync(base + on, h.nb.data(), h.nb.size() * sizeof(uint16_t), hipMemcpyHostToDevice, stream);
        if (e == hipSuccess) e = hipEventRecord(ev, stream);
        if (e != hipSuccess) {
            // nothing is published: wait for whatever was queued, then release it
            (void)hipStreamSynchronize(stream);
            if (ev) (void)hipEventDestroy(ev);
            if (base) (void)hipFree(base);
            return fail(SPA_ERR_HIP, "iq table %d upload: %s", idx, hipGetErrorString(e));
        }
        d.t.grid = base + og;
        d.t.map = (const int32_t*)(base + om);
        d.t.nb = (const uint16_t*)(base + on);
        d.t.size = kSpecs[idx].size;
        d.ready = ev;
    } else {
        SPA_HIP_TRY(hipStreamWaitEvent(stream, d.ready, 0));
    }
    *out = d.t;
    return 0;
}

}  // namespace spa

extern "C" int spa_iq_table_host(int index, const void** grid, int* grid_bytes, const int32_t** map, int* map_n,
                                 const uint16_t** neighbours, int* nb_n) {
    if (index < 0 || index > 5) return spa::fail(SPA_ERR_ARG, "spa_iq_table_host: index %d (0..5)", index);
    const spa::Host& h = spa::host_table(index);
    if (grid) *grid = h.grid.data();
    if (grid_bytes) *grid_bytes = (int)h.grid.size();
    if (map) *map = h.map.data();
    if (map_n) *map_n = (int)h.map.size();
    if (neighbours) *neighbours = h.nb.data();
    if (nb_n) *nb_n = (int)h.nb.size();
    return SPA_OK;
}
