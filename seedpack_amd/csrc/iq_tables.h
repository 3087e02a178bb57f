// Device copies of the IQ lattice tables (built once per process, uploaded once per device).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace spa {

struct IqDeviceTable {
    const uint8_t* grid;      // size x (8 or 4) coordinate values 2l+1
    const int32_t* map;       // level index -> grid point, or -1 - (offset << 9 | length) of its list in nb
    const uint16_t* nb;       // neighbour lists: count, then grid point indices
    int size;
};

// 0 IQ2_XXS, 1 IQ2_XS, 2 IQ1_S/IQ1_M, 3 IQ2_S, 4 IQ3_XXS, 5 IQ3_S; -1 otherwise
int iq_table_index(int ggml_type);
// the tables of `idx` on the current device; 0 or an SPA_ERR_* code. The first call on a device
// queues their upload on `stream`; work queued on `stream` after any call sees them complete.
int iq_device_table(int idx, IqDeviceTable* out, hipStream_t stream);

}  // namespace spa
