// Per-block phase stamps of the decode kernels: s_memrealtime (a 100 MHz counter shared by the whole device) at
// phase boundaries, written to the device array g_stamps at the end of each block.  Compiled in only with
// -DHY_STAMPS (python -m hyper_amd.build --stamps writes libhymoe_stamps.so); the default library has none of it.
// A stamped phase that ends in HY_STAMP_WAIT also waits for the wave's outstanding loads, which moves the first
// use's wait earlier: the timeline build runs slightly slower than the library it describes.
//   k_router_q8:     per wave at [4 gw]: entry, exit, kind (1 logit row, 2 Q8 of x)
//   k_route_gate_up: per block at [16384 + 8 b]: entry, routed, weights landed, dots done, fold done; [7] = 1
//   k_dec_down:      per block at [32768 + 8 b]: entry, slots, hidden quantized, weights landed, dots done, end; [7] = 1
#pragma once

#ifdef HY_STAMPS
namespace hy {
constexpr int STAMP_CAP = 1 << 16;
extern __device__ unsigned long long g_stamps[STAMP_CAP];
}
#define HY_STAMP_VARS(n) unsigned long long hy_st_[n] = {}
#define HY_STAMP(i) (hy_st_[i] = __builtin_amdgcn_s_memrealtime())
#define HY_STAMP_SET(i, v) (hy_st_[i] = (unsigned long long) (v))
#define HY_STAMP_WAIT(i)                                                                                               \
    do {                                                                                                               \
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");                                                               \
        HY_STAMP(i);                                                                                                   \
    } while (0)
// stamps 0 .. n-1 to g_stamps[base ..] (and 1 at base + 7 for the per-block records), by the calling lane if cond
#define HY_STAMP_SAVE(base, n, cond, flag)                                                                             \
    do {                                                                                                               \
        if ((cond) && (base) >= 0 && (base) + 8 <= STAMP_CAP) {                                                        \
            for (int i_ = 0; i_ < (n); ++i_) g_stamps[(base) + i_] = hy_st_[i_];                                       \
            if (flag) g_stamps[(base) + 7] = 1;                                                                        \
        }                                                                                                              \
    } while (0)
#else
#define HY_STAMP_VARS(n) do {} while (0)
#define HY_STAMP(i) do {} while (0)
#define HY_STAMP_SET(i, v) do {} while (0)
#define HY_STAMP_WAIT(i) do {} while (0)
#define HY_STAMP_SAVE(base, n, cond, flag) do {} while (0)
#endif
