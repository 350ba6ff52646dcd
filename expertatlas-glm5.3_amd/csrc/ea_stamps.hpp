// Per-block stage stamps for timelines of the decode layer and the small-row linear. They are compiled in only when
// EA_STAMPS is defined: `build.py --stamps` builds libea_exl3_stamps.so beside the product library, which is built
// without it and in which every mark below is empty. A mark stores the 100 MHz constant clock (s_memrealtime) of the
// marking thread into the region the host attached for the including file's kernels, at entry
// [block * STAMP_POINTS + point], with one plain vector store; point STAMP_POINTS - 1 holds a block descriptor instead
// of a time. Nothing is stored while no region is attached.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ea {

constexpr int STAMP_POINTS = 16;

#ifdef EA_STAMPS
static __device__ uint64_t* stamp_region;  // one a translation unit: the kernels of the file that includes this

__device__ __forceinline__ void stamp_value(int point, uint64_t v, bool who) {
    uint64_t* r = stamp_region;
    if (r && who) r[(size_t)blockIdx.x * STAMP_POINTS + point] = v;
}
// The host side: attach the region of the including file's kernels (nullptr detaches).
static inline int stamp_attach(void* region) {
    return hipMemcpyToSymbol(HIP_SYMBOL(stamp_region), &region, sizeof region) == hipSuccess ? 0 : -1;
}
// A mark: the time, or a value, stored by the threads for which `who` holds. In the product build the macros
// expand to nothing, so their arguments are not even evaluated and its code is what it is without them.
#define EA_STAMP(point, who) ::ea::stamp_value((point), __builtin_amdgcn_s_memrealtime(), (who))
#define EA_STAMP_VALUE(point, v, who) ::ea::stamp_value((point), (v), (who))
#else
#define EA_STAMP(point, who) ((void)0)
#define EA_STAMP_VALUE(point, v, who) ((void)0)
#endif

}  // namespace ea
