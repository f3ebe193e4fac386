// Internal interface between the C ABI (mbq_abi.cpp) and the kernel launchers (mbq_kernels.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace mbq {

enum : int { MBQ_BAD_ARG = -1, MBQ_LAUNCH_FAIL = -2, MBQ_SMALL_CAP = -3 };

// activation rows up to which the GEMV runs; more rows take the MFMA GEMM
constexpr int64_t GEMV_MAX_M = 4;

struct Args {
    const uint8_t* base;       // planes of the weight (layer already applied when the layer is a host value)
    int64_t stride;            // bytes between stacked weights (layer_dev)
    const int32_t* layer_dev;  // device layer index, or nullptr
    int nlayers;
    int64_t sc_off;            // offset of the scale plane inside one weight's planes
    int64_t hi_off, d_off;     // Q6_K: offsets of the high-bit plane and of the super-block scale plane
    int64_t wbytes;            // bytes of one weight's planes (int8: the N x K quants)
    const float* srow;         // int8: per-row scales
    const uint16_t* x;
    int64_t M, N, K;
    void* y;
    int out_bf16;
    bool noalloc = false;      // mbq_matmul_noalloc: split-K partials in the static scratch array, never allocated
};

// Split-K partials and arrival counters of the GEMM kernels, one set per device (mbq_gemm.hip): WS_BYTES of float32
// partial tiles and WS_TILES int counters, allocated (counters cleared) by the first call that needs them on a device
// and kept until the process ends. Every kernel that uses them leaves the counters it touched at zero.
constexpr size_t WS_BYTES = (size_t)64 << 20;
constexpr int WS_TILES = 1 << 16;
// the static scratch of mbq_matmul_noalloc: partial-tile bytes and arrival counters (automatic plans stay within it)
constexpr size_t SCRATCH_BYTES = (size_t)64 << 20;
constexpr int SCRATCH_TILES = 4096;
// fenced: the memory is ordinary cached memory (the static scratch of mbq_matmul_noalloc), so the blocks that exchange
// partials through it release and acquire at agent scope (split_release / split_acquire); the allocated workspace is
// uncached device memory, which no L2 holds, so its device-coherent stores and loads need no fence
struct Workspace { float* ws = nullptr; int* cnt = nullptr; size_t bytes = 0; int tiles = 0; int fenced = 0; };
int workspace(Workspace* out, hipStream_t s);   // refused while s is capturing and nothing is allocated yet
// The workspace of a split-K launch whose partial tiles take `bytes` over `tiles` arrival counters: the static scratch
// array when a.noalloc (mbq_matmul_noalloc; never allocated), else the allocated per-device workspace. An error, with
// nothing launched, when the plan does not fit it.
int split_workspace(const Args& a, int64_t tiles, size_t bytes, hipStream_t s, Workspace* out);

// largest weight plane or activation range a kernel addresses through a buffer resource (32-bit offsets; below the
// out-of-range offset OOB_VOFF of mbq_device.h)
constexpr int64_t BUF_MAX_BYTES = 0x7FFFFF00;

// records the calling thread's error message; returns code
int set_error(int code, const char* fmt, ...);

// Raises a kernel's dynamic-LDS limit to `lds` bytes on the current device, once per kernel (one `done` flag word per
// kernel) and device: the attribute belongs to the kernel on a device, so a process that launches on several GPUs sets
// it on each. Thread-safe; returns the HIP error of the first failing call.
inline hipError_t set_lds_limit(const void* kernel, size_t lds, std::atomic<uint64_t>& done) {
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
    const uint64_t bit = (dev >= 0 && dev < 64) ? (uint64_t{1} << dev) : 0;
    if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
    const hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_release);
    return e;
}

// compute units of the current device (cached per device; 256 if the query fails)
int cus_of_device();

int launch_matmul(int t, const Args& a, hipStream_t s);
int launch_gemv(int t, const Args& a, hipStream_t s);   // M <= GEMV_MAX_M (mbq_gemv.hip)
bool gemv_runs(int t, const Args& a);                   // the GEMV has a plan for this call (else the weight stream runs it)
// decode GEMV on 16-row tile planes (mbq_tgemv.hip), one activation row: launch_gemv and gemv_runs route tiled types
// there; it does not run while a GEMM kernel is forced (force_gemm_plan)
int launch_tgemv(int t, const Args& a, hipStream_t s);
bool tgemv_runs(int t, const Args& a);
int launch_gemm(int t, const Args& a, hipStream_t s);   // M > GEMV_MAX_M
// weight-stream GEMM (mbq_wsgemm.hip) for GEMV_MAX_M < M <= WS_MAX_M: rows_per_block 32 or 64, splits >= 1
constexpr int64_t WS_MAX_M = 64;
int launch_wsgemm(int t, const Args& a, int rows_per_block, int splits, hipStream_t s);
int wsgemm_plan(int t, const Args& a, int* rows_per_block, int* splits);
void wsgemm_effective(int t, const Args& a, int* rows_per_block, int* splits);   // what a launch with these runs
// K-group GEMM (mbq_kgemm.hip) of tiled planes (t = T_I8T or T_Q4KT) for M <= WS_MAX_M: splits = 0 chooses the K
// splits, else that many; the plan's rows per block and splits
int launch_kgemm(int t, const Args& a, int splits, hipStream_t s);
int kgemm_plan(int t, const Args& a, int splits, int* rows_per_block, int* chosen_splits);
// GEMM kernels (the values of MBQ_KERNEL_* in mbq.h)
enum : int { K_AUTO = 0, K_GEMV = 0, K_STREAM = 1, K_TILES = 2, K_KGROUP = 3 };
int gemm_plan(int t, const Args& a, int* kernel, int* bm, int* bn, int* splits);
int force_gemm_plan(int kernel, int bm, int bn, int splits);
int forced_gemm_kernel();                                 // the forced kernel, or K_AUTO
int launch_dequant(int t, const Args& a, float* w, const int32_t* rows, int64_t out_rows, hipStream_t s);   // rows: a row gather, or nullptr
int launch_int8_embed(const int8_t* q, const float* s, int64_t N, int64_t D, const int32_t* toks, int64_t T, void* y,
                      int out_bf16, hipStream_t st);
int launch_dequant_raw(int t, const uint8_t* raw, int64_t rows, int64_t K, float* w, hipStream_t s);
// the exact path's fused product for 1-8 activation rows on the file's blocks of an exact-only type (mbq_kernels.hip)
int launch_raw_gemv(int t, const uint8_t* raw, const uint16_t* x, int64_t M, int64_t N, int64_t K, void* y, int out_bf16,
                    hipStream_t s);
int launch_zero(uint8_t* p, int64_t n, hipStream_t s);   // n bytes at device address p set to zero
// measurement probes (mbq_probe.hip)
int launch_probe_read(const uint8_t* p, int64_t bytes, uint32_t* sink, hipStream_t s);
int launch_probe_mfma(int iters, float* sink, int64_t* flops, hipStream_t s);
int launch_probe_bf16(unsigned long long* diff, hipStream_t s);
struct Layout;
int launch_repack(int t, const uint8_t* raw, int64_t N, int64_t K, uint8_t* planes, const Layout& L, hipStream_t s);
// tiled int8 planes from the (N, K) int8 quants and (N,) float32 scales (padding rows and columns written as zero)
int launch_i8t_repack(const int8_t* q, const float* sc, int64_t N, int64_t K, uint8_t* planes, const Layout& L, hipStream_t s);

}  // namespace mbq
