// capi.hip -- the extern "C" boundary of libvcsrmc.so (declared in include/vcsrmc.h).
// Internal errors are C++ exceptions carrying a status; they stop here and become return
// codes, with the message kept per thread for vcsrmc_last_error().
#include <cstdio>
#include <mutex>
#include <new>
#include <string>

#include "../../include/vcsrmc.h"
#include "internal.hpp"

struct vcsrmc_format_s {
    vcsrmc::DeviceFormat F;
    int device = 0;
};

namespace vcsrmc {

[[noreturn]] void throw_hip(hipError_t e, const char* what, const char* file, int line) {
    char buf[512];
    std::snprintf(buf, sizeof buf, "HIP error %s (%s) in %s at %s:%d", hipGetErrorName(e),
                  hipGetErrorString(e), what, file, line);
    throw Error(VCSRMC_ERR_HIP, buf);
}

}  // namespace vcsrmc

// Scratch of vcsrmc_spmm_noalloc: a static device array, one copy per GPU.  In host code the
// name `scratch` is only a stand-in for the symbol, never a device address: the copy of the
// current device is reached through the address hipGetSymbolAddress returns for it.
static __device__ __attribute__((aligned(256))) unsigned char scratch[VCSRMC_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_last_error;

template <typename Fn>
int guarded(Fn&& fn) {
    try {
        fn();
        return VCSRMC_OK;
    } catch (const vcsrmc::Error& e) {
        g_last_error = e.what();
        return e.status;
    } catch (const std::bad_alloc&) {
        g_last_error = "host allocation failed";
        return VCSRMC_ERR_HIP;
    } catch (const std::exception& e) {
        g_last_error = e.what();
        return VCSRMC_ERR_HIP;
    }
}

// Makes the handle's device current for the scope of a call.
struct DeviceScope {
    int prev = -1;
    explicit DeviceScope(int dev) {
        VCSRMC_HIP(hipGetDevice(&prev));
        if (prev != dev) VCSRMC_HIP(hipSetDevice(dev));
    }
    ~DeviceScope() {
        int cur = -1;
        if (hipGetDevice(&cur) == hipSuccess && cur != prev && prev >= 0) (void)hipSetDevice(prev);
    }
};

void need(bool ok, const char* msg) {
    if (!ok) throw vcsrmc::Error(VCSRMC_ERR_ARG, msg);
}

// The copy of `scratch` (below) on each device, looked up once per device.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's scratch (the caller has made `dev` current).
void* scratch_of_device(int dev) {
    if (dev < 0 || dev >= kMaxDevices) throw vcsrmc::Error(VCSRMC_ERR_ARG, "device index too large");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        VCSRMC_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        if (!ptr) throw vcsrmc::Error(VCSRMC_ERR_HIP, "no device address for the scratch array");
        g_scratch_ptr[dev] = ptr;
    }
    return g_scratch_ptr[dev];
}

}  // namespace

extern "C" {

int vcsrmc_create(vcsrmc_t* out) {
    return guarded([&] {
        need(out != nullptr, "null output handle");
        *out = nullptr;
        auto* h = new vcsrmc_format_s();
        if (hipGetDevice(&h->device) != hipSuccess) {
            delete h;
            throw vcsrmc::Error(VCSRMC_ERR_HIP, "no HIP device");
        }
        *out = h;
    });
}

int vcsrmc_destroy(vcsrmc_t h) {
    return guarded([&] {
        if (!h) return;
        {
            DeviceScope ds(h->device);
            h->F.clear();
        }
        delete h;
    });
}

int vcsrmc_half_scale(const float* d_val, long long nnz, float* scale, void* stream) {
    return guarded([&] {
        need(scale != nullptr && nnz >= 0 && (nnz == 0 || d_val != nullptr), "bad argument");
        const float amax = vcsrmc::device_absmax(d_val, nnz, (hipStream_t)stream);
        *scale = vcsrmc::half_scale_from_amax(amax);
    });
}

int vcsrmc_rcm_order(const int* d_row_ptr, const int* d_col, int M, int N, int nnz,
                     int* d_position, void* stream) {
    return guarded([&] {
        vcsrmc::rcm_order_device(d_row_ptr, d_col, M, N, nnz, d_position, (hipStream_t)stream);
    });
}

int vcsrmc_set_rcm_limits(long long max_levels, long long max_rounds) {
    return guarded([&] {
        need(max_levels >= 0 && max_rounds >= 0, "negative limit");
        vcsrmc::set_rcm_limits(max_levels, max_rounds);
    });
}

int vcsrmc_set_row_grouping(int mode) {
    return guarded([&] {
        need(mode >= 0 && mode <= 2, "row grouping mode must be 0, 1 or 2");
        vcsrmc::set_row_grouping(mode);
    });
}

int vcsrmc_set_fp32_row_steps(int mode) {
    return guarded([&] {
        need(mode >= 0 && mode <= 2, "FP32 row-step mode must be 0, 1 or 2");
        vcsrmc::set_fp32_row_steps(mode);
    });
}

int vcsrmc_apply_column_permutation(const int* d_row_ptr, int* d_col, float* d_val, int M, int N,
                                    int nnz, const int* d_position, const float* d_B, int O,
                                    float* d_B_out, void* stream) {
    return guarded([&] {
        vcsrmc::apply_column_permutation_device(d_row_ptr, d_col, d_val, M, N, nnz, d_position,
                                                d_B, O, d_B_out, (hipStream_t)stream);
    });
}

int vcsrmc_build_csr(vcsrmc_t h, const int* d_row_ptr, const int* d_col, const float* d_val,
                     int M, int N, int nnz, int fp32, int segw, void* stream) {
    return guarded([&] {
        need(h != nullptr, "null handle");
        DeviceScope ds(h->device);
        try {
            vcsrmc::build_from_csr(h->F, d_row_ptr, d_col, d_val, M, N, nnz, segw, fp32,
                                   (hipStream_t)stream);
        } catch (...) {
            h->F.clear();
            throw;
        }
    });
}

int vcsrmc_upload(vcsrmc_t h, int M, int N, int segw, int bundle, int num_segments,
                  int num_groups, long long nval, int num_items, const int* group_ptr,
                  const int* group_depth, const int* group_seg_base, const int* group_rows,
                  const int* lcol, const float* val, const int* item_gbeg, const int* item_gend,
                  float scale, int fp32, void* stream) {
    return guarded([&] {
        need(h != nullptr, "null handle");
        need(group_ptr != nullptr, "null group_ptr");
        DeviceScope ds(h->device);
        vcsrmc::HostArrays H{M, N, segw, bundle, num_segments, num_groups, num_items, nval,
                             group_ptr, group_depth, group_seg_base, group_rows, lcol, val,
                             item_gbeg, item_gend, scale, fp32};
        try {
            vcsrmc::build_from_host(h->F, H, (hipStream_t)stream);
        } catch (...) {
            h->F.clear();
            throw;
        }
    });
}

int vcsrmc_get_info(vcsrmc_t h, vcsrmc_info* out) {
    return guarded([&] {
        need(h != nullptr && out != nullptr, "null argument");
        if (!h->F.ready) throw vcsrmc::Error(VCSRMC_ERR_STATE, "no format in this handle");
        const auto& F = h->F;
        out->M = F.M; out->N = F.N; out->segw = F.segw; out->bundle = F.bundle;
        out->num_segments = F.num_segments; out->num_groups = F.G; out->nval = F.nval;
        out->num_items = F.nitems; out->scale = F.scale; out->fp32 = F.fp32; out->nnz = F.nnz;
        out->num_panels = F.num_panels; out->num_chunks = F.num_chunks;
        out->num_units = F.num_units; out->device = h->device;
        out->num_dense = F.num_dense;
        out->row_grouped = F.row_map.n > 0;
        out->num_heavy = F.num_heavy;
        out->num_split_panels = F.num_split_panels;
        out->num_row_step_batches = F.num_row_step_batches;
    });
}

int vcsrmc_get_row_map(vcsrmc_t h, int* row_of_position, long long capacity, long long* length) {
    return guarded([&] {
        need(h != nullptr && length != nullptr, "null argument");
        if (!h->F.ready) throw vcsrmc::Error(VCSRMC_ERR_STATE, "no format in this handle");
        const auto& F = h->F;
        *length = (long long)F.row_map.n;
        if (F.row_map.n == 0 || row_of_position == nullptr) return;
        need(capacity >= (long long)F.row_map.n, "row map buffer smaller than its length");
        DeviceScope ds(h->device);
        VCSRMC_HIP(hipMemcpy(row_of_position, F.row_map.p, sizeof(int) * F.row_map.n,
                             hipMemcpyDeviceToHost));
    });
}

int vcsrmc_get_units(vcsrmc_t h, int* units, long long capacity, long long* num_units,
                     int* xcd_start) {
    return guarded([&] {
        need(h != nullptr && num_units != nullptr, "null argument");
        if (!h->F.ready) throw vcsrmc::Error(VCSRMC_ERR_STATE, "no format in this handle");
        const auto& F = h->F;
        *num_units = F.num_units;
        if (xcd_start)
            for (int x = 0; x < 9; ++x) xcd_start[x] = F.xcd_start[x];
        if (units == nullptr || F.num_units == 0) return;
        need(capacity >= 4LL * F.num_units, "units buffer smaller than 4 ints per unit");
        DeviceScope ds(h->device);
        VCSRMC_HIP(hipMemcpy(units, F.units.p, sizeof(int4) * (size_t)F.num_units,
                             hipMemcpyDeviceToHost));
    });
}

int vcsrmc_traffic_floor(vcsrmc_t h, int b_dtype, int O, int tileK, int flags,
                         vcsrmc_traffic* out, void* stream) {
    return guarded([&] {
        need(h != nullptr && out != nullptr, "null argument");
        need(b_dtype == VCSRMC_B_F32 || b_dtype == VCSRMC_B_F16, "unknown B dtype");
        need((flags & ~VCSRMC_SPMM_OVERWRITE) == 0, "unknown flag");
        DeviceScope ds(h->device);
        const vcsrmc::TrafficFloor t =
            vcsrmc::traffic_floor(h->F, b_dtype == VCSRMC_B_F16, O, tileK,
                                  !(flags & VCSRMC_SPMM_OVERWRITE), (hipStream_t)stream);
        out->b_bytes = t.b_bytes;
        out->b_once_bytes = t.b_once_bytes;
        out->a_bytes = t.a_bytes;
        out->c_bytes = t.c_bytes;
        out->convert_bytes = t.convert_bytes;
        out->total = t.total;
        out->o_tile_width = t.o_tile_width;
        out->o_tiles = t.o_tiles;
        out->row_parts = t.row_parts;
    });
}

int vcsrmc_download(vcsrmc_t h, int* group_ptr, int* group_depth, int* group_seg_base,
                    int* group_rows, int* lcol, float* val, int* item_gbeg, int* item_gend) {
    return guarded([&] {
        need(h != nullptr, "null handle");
        if (!h->F.ready) throw vcsrmc::Error(VCSRMC_ERR_STATE, "no format in this handle");
        DeviceScope ds(h->device);
        const auto& F = h->F;
        auto get = [](void* dst, const void* src, size_t bytes) {
            if (dst && bytes) VCSRMC_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
        };
        get(group_ptr, F.group_ptr.p, sizeof(int) * ((size_t)F.G + 1));
        get(group_depth, F.group_depth.p, sizeof(int) * (size_t)F.G);
        get(group_seg_base, F.group_seg_base.p, sizeof(int) * (size_t)F.G);
        get(group_rows, F.group_rows.p, sizeof(int) * 16 * (size_t)F.G);
        get(lcol, F.lcol.p, sizeof(int) * (size_t)F.nval);
        get(val, F.val.p, sizeof(float) * (size_t)F.nval);
        get(item_gbeg, F.item_gbeg.p, sizeof(int) * (size_t)F.nitems);
        get(item_gend, F.item_gend.p, sizeof(int) * (size_t)F.nitems);
    });
}

int vcsrmc_spmm(vcsrmc_t h, const void* dB, int b_dtype, int O, int tileK, float* dC,
                void* stream, float* ms) {
    return vcsrmc_spmm_ex(h, dB, b_dtype, O, tileK, dC, 0, stream, ms);
}

int vcsrmc_spmm_ex(vcsrmc_t h, const void* dB, int b_dtype, int O, int tileK, float* dC,
                   int flags, void* stream, float* ms) {
    return guarded([&] {
        need(h != nullptr, "null handle");
        need(b_dtype == VCSRMC_B_F32 || b_dtype == VCSRMC_B_F16, "unknown B dtype");
        need((flags & ~VCSRMC_SPMM_OVERWRITE) == 0, "unknown flag");
        const bool accumulate = !(flags & VCSRMC_SPMM_OVERWRITE);
        DeviceScope ds(h->device);
        hipStream_t st = (hipStream_t)stream;
        if (!ms) {
            vcsrmc::spmm_launch(h->F, dB, b_dtype == VCSRMC_B_F16, O, tileK, dC, accumulate, st);
            return;
        }
        hipEvent_t t0, t1;
        VCSRMC_HIP(hipEventCreate(&t0));
        VCSRMC_HIP(hipEventCreate(&t1));
        try {
            // host decisions first: the events bracket the enqueued kernels only
            const vcsrmc::SpmmPlan plan =
                vcsrmc::plan_spmm(h->F, dB, b_dtype == VCSRMC_B_F16, O, tileK, dC, accumulate);
            VCSRMC_HIP(hipEventRecord(t0, st));
            vcsrmc::run_spmm(plan, st);
            VCSRMC_HIP(hipEventRecord(t1, st));
            VCSRMC_HIP(hipEventSynchronize(t1));
            VCSRMC_HIP(hipEventElapsedTime(ms, t0, t1));
        } catch (...) {
            (void)hipEventDestroy(t0);
            (void)hipEventDestroy(t1);
            throw;
        }
        VCSRMC_HIP(hipEventDestroy(t0));
        VCSRMC_HIP(hipEventDestroy(t1));
    });
}

int vcsrmc_spmm_noalloc(vcsrmc_t h, const void* dB, int b_dtype, int O, int tileK, float* dC,
                        int flags, void* stream) {
    return guarded([&] {
        need(h != nullptr, "null handle");
        need(b_dtype == VCSRMC_B_F32 || b_dtype == VCSRMC_B_F16, "unknown B dtype");
        need((flags & ~VCSRMC_SPMM_OVERWRITE) == 0, "unknown flag");
        DeviceScope ds(h->device);
        vcsrmc::HalfScratch ext;
        ext.p = static_cast<_Float16*>(scratch_of_device(h->device));
        ext.halves = VCSRMC_NOALLOC_SCRATCH_BYTES / sizeof(_Float16);
        vcsrmc::spmm_launch(h->F, dB, b_dtype == VCSRMC_B_F16, O, tileK, dC,
                            !(flags & VCSRMC_SPMM_OVERWRITE), (hipStream_t)stream, ext);
    });
}

const char* vcsrmc_status_string(int status) {
    switch (status) {
        case VCSRMC_OK: return "ok";
        case VCSRMC_ERR_ARG: return "invalid argument";
        case VCSRMC_ERR_SEGW: return "vcsr_mc supports segw in {16, 32, 48, 64}";
        case VCSRMC_ERR_TILEK: return "vcsr_mc supports tileK in {16, 32, 64, 128}";
        case VCSRMC_ERR_CSR: return "invalid CSR";
        case VCSRMC_ERR_UNSORTED: return "CSR columns not strictly increasing within a row";
        case VCSRMC_ERR_FORMAT: return "inconsistent format arrays";
        case VCSRMC_ERR_OVERFLOW: return "format size exceeds int32";
        case VCSRMC_ERR_HIP: return "HIP runtime error";
        case VCSRMC_ERR_STATE: return "no format";
        case VCSRMC_ERR_SCRATCH: return "input exceeds the static scratch of vcsrmc_spmm_noalloc";
        default: return "unknown status";
    }
}

const char* vcsrmc_last_error(void) { return g_last_error.c_str(); }

}  // extern "C"
