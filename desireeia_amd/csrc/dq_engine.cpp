// dq_engine.cpp - the engine-facing GPU operator entry points (the GPU block of
// the reference's core/engine.h:502-811) over the kernel layer of this library.
//
// Host code only. State is process-global, as in the reference backend
// (cuda/backend_cuda.cu): one stream, scratch buffers that grow on demand, the
// device KV cache, the x vectors a chain of layers passes along, a registry
// of the uploaded weight matrices, and (optionally) one HIP graph per layer.
//
// Conventions (core/engine.h, models/dense_forward.cpp:327-366):
//  * NOT_SUPPORTED means "not covered here": nothing is written to the
//    caller's outputs and the engine recomputes on the CPU. Every such check
//    runs before any device work.
//  * IO means a device failure; the sticky error is cleared so the engine's
//    CPU fallback and later calls are not poisoned.
//  * Calls returning host data synchronise the stream once; a chain of
//    cuda_layer_forward calls synchronises only where download_x is set.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <unordered_map>
#include <vector>

#include "../../include/desireeia_hip.h"
#include "dq_common.h"

namespace {

// ------------------------------------------------------------------ state --

struct DevBuf {
    void* p = nullptr;
    size_t cap = 0;
};

struct WInfo {
    int fmt;
    size_t rows, cols;
    const void* base;  // == the key for a matrix; the matrix for a Q8_0 scale view
    void* tiles;       // the prefill GEMM's tile copy (DESIREEIA_GEMM_TILES), or NULL
};

struct LayerGraph {
    hipGraphExec_t exec = nullptr;
    const void* key[7];
    float* x_in;
    float* x_out;
    size_t work_bytes;
};

struct Engine {
    hipStream_t stream = nullptr;
    DevBuf xbuf, ybuf, act, work, stage;
    DevBuf lx[2];        // layer chain x ping-pong
    int cur = 0;         // lx[cur] holds the current x
    DevBuf rope;         // RoPE table of the current token
    DevBuf rope_all;     // per-layer slots: the RoPE tables of every layer
    size_t rope_all_n = 0;  // floats of rope_all uploaded (0: none)
    bool rope_on = false;
    uint8_t* kc = nullptr;
    uint8_t* vc = nullptr;
    size_t kv_bytes = 0;
    std::unordered_map<const void*, WInfo> reg;
    std::unordered_map<const void*, LayerGraph> graphs;  // keyed by wq
    // prefill: the prompt's activations, RoPE table slots, the layer
    // workspace and norm weights, and the K/V rows still to be mirrored to
    // the host cache (copied with the prompt's one synchronisation)
    DevBuf px, prope[4], pwork, pnorm, pio;
    struct Mirror {
        uint8_t* k;
        uint8_t* v;
        size_t off, bytes;
    };
    std::vector<Mirror> mirror;
    // output head and the pipelined draw: logits, top-k, the model's output
    // norm (device copy, re-sent when its content changes), the draw state,
    // pinned readback slots with an event each and the readback stream
    DevBuf hlog, hwork, htk, hnorm, hcand;
    std::vector<float> hnorm_host;
    dq_sample_state_t* sst = nullptr;
    int32_t* tok_pinned = nullptr;
    hipEvent_t tok_ev[4] = {}, drawn_ev[4] = {};
    hipStream_t tok_stream = nullptr;
};

Engine g;

int io_fail() {
    (void)hipGetLastError();
    return DQ_ERR_IO;
}

hipStream_t stream() {
    if (!g.stream && hipStreamCreate(&g.stream) != hipSuccess) {
        (void)hipGetLastError();
        g.stream = nullptr;
    }
    return g.stream;
}

void drop_graphs() {
    for (auto& kv : g.graphs)
        if (kv.second.exec) (void)hipGraphExecDestroy(kv.second.exec);
    g.graphs.clear();
}

// Grows b to at least n bytes. Pending work on the stream may still use the
// old buffer (a chain of layers is not synchronised between calls), so the
// stream drains first; captured graphs hold the old address and are dropped.
bool reserve(DevBuf& b, size_t n) {
    if (n <= b.cap && b.p) return true;
    if (g.stream) (void)hipStreamSynchronize(g.stream);
    drop_graphs();
    if (b.p) (void)hipFree(b.p);
    b.p = nullptr;
    b.cap = 0;
    const size_t want = n < 256 ? 256 : n;
    if (hipMalloc(&b.p, want) != hipSuccess) {
        (void)hipGetLastError();
        b.p = nullptr;
        return false;
    }
    b.cap = want;
    return true;
}

void release(DevBuf& b) {
    if (b.p) (void)hipFree(b.p);
    b.p = nullptr;
    b.cap = 0;
}

int sync() { return hipStreamSynchronize(g.stream) == hipSuccess ? DQ_OK : io_fail(); }

bool env_flag(const char* name) {
    const char* e = getenv(name);
    return e && *e && strcmp(e, "0") != 0;
}

// ------------------------------------------------------------ activations --

// Quantized activation triple carved from one scratch buffer.
struct Act {
    int8_t* q;
    float* s;
    int32_t* i;
};

size_t act_bytes(size_t cols) { return dq_align256(cols) + 2 * dq_align256(cols / 32 * 4); }

Act carve_act(uint8_t* base, size_t cols) {
    Act a;
    a.q = (int8_t*)base;
    a.s = (float*)(base + dq_align256(cols));
    a.i = (int32_t*)(base + dq_align256(cols) + dq_align256(cols / 32 * 4));
    return a;
}

int act_kind(int fmt) { return (fmt == DQ_FMT_Q8_0 || fmt == DQ_FMT_Q4_0) ? DQ_ACT_Q8_0 : DQ_ACT_Q8K_REP; }

bool fmt_ok(int fmt) {
    return fmt == DQ_FMT_Q8_0 || fmt == DQ_FMT_Q4_0 || fmt == DQ_FMT_Q4_K || fmt == DQ_FMT_Q6_K;
}

// The activation quantizer needs cols % 32 (per 32) or % 256 (per 256); the
// GEMV's packed layouts need cols % 64 (Q8_0, Q4_0) or % 256 (K-quants), and
// at most 8 items of 64 per lane (cols <= 131072 with the 4-way K split).
bool gemv_shape_ok(int fmt, size_t rows, size_t cols) {
    DqLayout L;
    return fmt_ok(fmt) && rows > 0 && rows <= 0x3FFFFFFF && cols > 0 && cols <= 131072 &&
           dq_layout(fmt, rows, cols, &L);
}

// Looks a matrix up; NULL if it was not uploaded here.
const WInfo* lookup(const void* p) {
    auto it = g.reg.find(p);
    return it == g.reg.end() ? nullptr : &it->second;
}

// ------------------------------------------------------------- GEMV core --

// x (host, cols floats) -> device; every job's GEMV (the activation quantized
// in-kernel, or once per activation kind for very wide rows) into device y
// slices, then the host copies and one synchronisation. jobs: (fmt, d_w,
// rows) with host y.
struct HostJob {
    int fmt;
    const void* d_w;
    size_t rows;
    float* y;
};

int run_host_jobs(const HostJob* jobs, size_t n, size_t cols, const float* x) {
    if (n == 0) return DQ_OK;
    if (!x) return DQ_ERR_INVALID_ARG;
    size_t total_rows = 0;
    bool need[2] = {false, false};
    for (size_t j = 0; j < n; ++j) {
        if (!jobs[j].d_w || !jobs[j].y || !gemv_shape_ok(jobs[j].fmt, jobs[j].rows, cols))
            return DQ_ERR_NOT_SUPPORTED;
        if (act_kind(jobs[j].fmt) == DQ_ACT_Q8K_REP && cols % 256) return DQ_ERR_NOT_SUPPORTED;
        need[act_kind(jobs[j].fmt)] = true;
        total_rows += jobs[j].rows;
    }
    if (!stream()) return DQ_ERR_IO;
    if (!reserve(g.xbuf, cols * 4) || !reserve(g.act, 2 * act_bytes(cols)) || !reserve(g.ybuf, total_rows * 4))
        return DQ_ERR_IO;
    const hipStream_t s = g.stream;
    float* dx = (float*)g.xbuf.p;
    if (hipMemcpyAsync(dx, x, cols * 4, hipMemcpyHostToDevice, s) != hipSuccess) return io_fail();
    float* dy = (float*)g.ybuf.p;
    std::vector<float*> ys(n);
    size_t off = 0;
    for (size_t j = 0; j < n; ++j) {
        ys[j] = dy + off;
        off += jobs[j].rows;
    }
    if (cols <= 49152) {
        // the GEMVs quantize x in-kernel: grouped launches of up to 4 jobs
        dq_gemv_job_t grp[4];
        for (size_t j0 = 0; j0 < n; j0 += 4) {
            const size_t m = n - j0 < 4 ? n - j0 : 4;
            for (size_t j = 0; j < m; ++j)
                grp[j] = {jobs[j0 + j].fmt, jobs[j0 + j].d_w, jobs[j0 + j].rows, ys[j0 + j], nullptr};
            const int rc = dq_gemv_group_f32(grp, m, cols, dx, s);
            if (rc != DQ_OK) return rc == DQ_ERR_IO ? io_fail() : rc;
        }
        for (size_t j = 0; j < n; ++j)
            if (hipMemcpyAsync(jobs[j].y, ys[j], jobs[j].rows * 4, hipMemcpyDeviceToHost, s) != hipSuccess)
                return io_fail();
        return sync();
    }
    // wider rows: quantize once per activation kind, then grouped GEMVs
    Act a[2] = {carve_act((uint8_t*)g.act.p, cols), carve_act((uint8_t*)g.act.p + act_bytes(cols), cols)};
    for (int k = 0; k < 2; ++k)
        if (need[k]) {
            const int rc = dq_quantize_act(k, dx, cols, 1, a[k].q, a[k].s, a[k].i, nullptr, s);
            if (rc != DQ_OK) return rc == DQ_ERR_IO ? io_fail() : rc;
        }
    for (int k = 0; k < 2; ++k) {
        dq_gemv_job_t grp[4];
        int m = 0;
        for (size_t j = 0; j <= n; ++j) {
            if (j < n && act_kind(jobs[j].fmt) == k) grp[m++] = {jobs[j].fmt, jobs[j].d_w, jobs[j].rows, ys[j], nullptr};
            if (m == 4 || (j == n && m > 0)) {
                const int rc = dq_gemv_group(grp, (size_t)m, cols, a[k].q, a[k].s, a[k].i, s);
                if (rc != DQ_OK) return rc == DQ_ERR_IO ? io_fail() : rc;
                m = 0;
            }
        }
    }
    for (size_t j = 0; j < n; ++j)
        if (hipMemcpyAsync(jobs[j].y, ys[j], jobs[j].rows * 4, hipMemcpyDeviceToHost, s) != hipSuccess) return io_fail();
    return sync();
}

// --------------------------------------------------------------- uploads --

bool upload_packed(int fmt, const uint8_t* data, size_t rows, size_t cols, void** out) {
    *out = nullptr;
    DqLayout L;
    if (!data || rows == 0 || !dq_layout(fmt, rows, cols, &L)) return false;
    if (!stream()) return false;
    const size_t gguf = rows * dq_gguf_row_bytes(fmt, cols);
    void* dev = nullptr;
    if (hipMalloc(&dev, L.total) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    // the GGUF rows go through the staging buffer and are repacked on the device
    if (!reserve(g.stage, gguf) ||
        hipMemcpyAsync(g.stage.p, data, gguf, hipMemcpyHostToDevice, g.stream) != hipSuccess ||
        dq_weights_pack(fmt, g.stage.p, rows, cols, dev, g.stream) != DQ_OK ||
        hipStreamSynchronize(g.stream) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(dev);
        return false;
    }
    // opt-in (DESIREEIA_GEMM_TILES=1): a tile copy for the prefill GEMMs
    // beside the packed rows the decode GEMV reads (the weights held twice)
    void* tiles = nullptr;
    const bool want_tiles = env_flag("DESIREEIA_GEMM_TILES");  // read per upload
    size_t tb = 0;
    if (want_tiles && cols % 256 == 0 && dq_gemm_tiles_bytes(fmt, rows, cols, &tb) == DQ_OK) {
        if (hipMalloc(&tiles, tb) != hipSuccess) {
            (void)hipGetLastError();
            tiles = nullptr;
        } else if (dq_gemm_tiles_pack(fmt, dev, rows, cols, tiles, g.stream) != DQ_OK ||
                   hipStreamSynchronize(g.stream) != hipSuccess) {
            (void)hipGetLastError();
            (void)hipFree(tiles);
            tiles = nullptr;
        }
    }
    g.reg[dev] = WInfo{fmt, rows, cols, dev, tiles};
    *out = dev;
    return true;
}

// ------------------------------------------------------------- KV / layer --

size_t kv_pos_bytes(uint32_t n_head_kv, uint32_t head_dim) { return (size_t)n_head_kv * (head_dim / 32) * DQ_SZ_Q8_0; }

// Positions of the layer at byte offset `off` that fit in the device cache.
uint32_t kv_positions(size_t off, size_t pos_bytes) {
    if (!g.kc || off >= g.kv_bytes || pos_bytes == 0) return 0;
    const size_t n = (g.kv_bytes - off) / pos_bytes;
    return n > 0x7FFFFFFF ? 0x7FFFFFFF : (uint32_t)n;
}

int upload_rope(const float* rope_cache, uint32_t n_rot) {
    if (!reserve(g.rope, 512 * 4)) return DQ_ERR_IO;
    g.rope_on = rope_cache != nullptr;
    if (rope_cache &&
        hipMemcpyAsync(g.rope.p, rope_cache, (size_t)n_rot * 4, hipMemcpyHostToDevice, g.stream) != hipSuccess)
        return io_fail();
    return DQ_OK;
}

}  // namespace

extern "C" {

// ---------------------------------------------------------------- devices --

int32_t cuda_gpu_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();  // no driver / no device: not an error for the caller
        return 0;
    }
    return n;
}

bool cuda_probe_gpu(int32_t index, char* name, size_t name_len, uint64_t* total, uint64_t* free_bytes,
                    int32_t* cc_major, int32_t* cc_minor, int32_t* sms) {
    if (index < 0 || index >= cuda_gpu_count() || !total || !free_bytes || !cc_major || !cc_minor || !sms)
        return false;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, index) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    if (name && name_len) snprintf(name, name_len, "%s", prop.name);
    *cc_major = prop.major;
    *cc_minor = prop.minor;
    *sms = prop.multiProcessorCount;
    *total = prop.totalGlobalMem;
    *free_bytes = 0;
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess) prev = 0;
    if (hipSetDevice(index) == hipSuccess) {
        size_t f = 0, t = 0;
        if (hipMemGetInfo(&f, &t) == hipSuccess) {
            *free_bytes = f;
            *total = t;
        }
        (void)hipSetDevice(prev);
    }
    (void)hipGetLastError();
    return true;
}

// ---------------------------------------------------------------- uploads --

bool matmul_q8_0_cuda_upload_weights(const uint8_t* q8_data, size_t rows, size_t cols, void** out_d_qs,
                                     void** out_d_scale) {
    if (!out_d_qs || !out_d_scale) return false;
    *out_d_qs = *out_d_scale = nullptr;
    void* dev = nullptr;
    if (!upload_packed(DQ_FMT_Q8_0, q8_data, rows, cols, &dev)) return false;
    DqLayout L;
    dq_layout(DQ_FMT_Q8_0, rows, cols, &L);
    // the scale plane of the packed matrix, handed out as the engine's
    // separate scale pointer (a view: freeing it frees nothing)
    void* view = (uint8_t*)dev + L.d_off;
    g.reg[view] = WInfo{DQ_FMT_Q8_0, rows, cols, dev, nullptr};
    *out_d_qs = dev;
    *out_d_scale = view;
    return true;
}

bool cuda_upload_weights(int format, const uint8_t* data, size_t rows, size_t cols, void** out_d_qs,
                         void** out_d_scale) {
    if (!out_d_qs || !out_d_scale) return false;
    *out_d_qs = *out_d_scale = nullptr;
    if (format == DQ_FMT_Q8_0) return matmul_q8_0_cuda_upload_weights(data, rows, cols, out_d_qs, out_d_scale);
    if (format != DQ_FMT_Q4_0 && format != DQ_FMT_Q4_K && format != DQ_FMT_Q6_K) return false;
    return upload_packed(format, data, rows, cols, out_d_qs);
}

void cuda_free_device(void* p) {
    if (!p) return;
    auto it = g.reg.find(p);
    if (it != g.reg.end() && it->second.base != p) {  // a Q8_0 scale view
        g.reg.erase(it);
        return;
    }
    // graphs that read this matrix are dropped with it
    for (auto gi = g.graphs.begin(); gi != g.graphs.end();) {
        bool uses = false;
        for (const void* k : gi->second.key) uses = uses || k == p;
        if (uses) {
            (void)hipGraphExecDestroy(gi->second.exec);
            gi = g.graphs.erase(gi);
        } else {
            ++gi;
        }
    }
    void* tiles = it != g.reg.end() ? it->second.tiles : nullptr;
    if (it != g.reg.end()) g.reg.erase(it);
    if (g.stream) (void)hipStreamSynchronize(g.stream);
    if (tiles) (void)hipFree(tiles);
    (void)hipFree(p);
    (void)hipGetLastError();
}

void cuda_backend_shutdown(void) {
    if (g.stream) (void)hipStreamSynchronize(g.stream);
    drop_graphs();
    for (DevBuf* b : {&g.xbuf, &g.ybuf, &g.act, &g.work, &g.stage, &g.lx[0], &g.lx[1], &g.rope, &g.rope_all, &g.px,
                      &g.prope[0], &g.prope[1], &g.prope[2], &g.prope[3], &g.pwork, &g.pnorm, &g.pio, &g.hlog,
                      &g.hwork, &g.htk, &g.hnorm, &g.hcand})
        release(*b);
    g.rope_all_n = 0;
    g.mirror.clear();
    g.hnorm_host.clear();
    if (g.tok_stream) (void)hipStreamSynchronize(g.tok_stream);
    for (int i = 0; i < 4; ++i) {
        if (g.tok_ev[i]) (void)hipEventDestroy(g.tok_ev[i]);
        if (g.drawn_ev[i]) (void)hipEventDestroy(g.drawn_ev[i]);
        g.tok_ev[i] = g.drawn_ev[i] = nullptr;
    }
    if (g.tok_stream) (void)hipStreamDestroy(g.tok_stream);
    g.tok_stream = nullptr;
    if (g.sst) (void)hipFree(g.sst);
    g.sst = nullptr;
    if (g.tok_pinned) (void)hipHostFree(g.tok_pinned);
    g.tok_pinned = nullptr;
    cuda_kv_cache_release();
    if (g.stream) (void)hipStreamDestroy(g.stream);
    g.stream = nullptr;
    g.cur = 0;
    (void)hipGetLastError();
}

// ------------------------------------------------------------------ GEMVs --

int matmul_kquant_cuda_resident(int format, const void* d_w, size_t rows, size_t cols, const float* x, float* y) {
    if (format == DQ_FMT_Q8_0) return DQ_ERR_NOT_SUPPORTED;  // Q8_0 goes through matmul_q8_0_cuda_resident
    const HostJob j = {format, d_w, rows, y};
    return run_host_jobs(&j, 1, cols, x);
}

int matmul_kquant_cuda_resident_same_x(const CudaKQuantJob* jobs, size_t n, size_t cols, const float* x) {
    if (n && !jobs) return DQ_ERR_INVALID_ARG;
    std::vector<HostJob> hj(n);
    for (size_t j = 0; j < n; ++j) {
        if (jobs[j].format == DQ_FMT_Q8_0) return DQ_ERR_NOT_SUPPORTED;
        hj[j] = {jobs[j].format, jobs[j].d_w, jobs[j].rows, jobs[j].y};
    }
    return run_host_jobs(hj.data(), n, cols, x);
}

int matmul_q8_0_cuda_resident(const void* d_qs, const void* d_scale, size_t rows, size_t cols, const float* x,
                              float* y) {
    if (!d_qs || !d_scale) return DQ_ERR_NOT_SUPPORTED;
    const HostJob j = {DQ_FMT_Q8_0, d_qs, rows, y};
    return run_host_jobs(&j, 1, cols, x);
}

int matmul_q8_0_cuda_resident_group(const CudaQ80Job* jobs, size_t n, size_t cols, const float* x) {
    if (n && !jobs) return DQ_ERR_INVALID_ARG;
    std::vector<HostJob> hj(n);
    for (size_t j = 0; j < n; ++j) {
        if (!jobs[j].d_qs || !jobs[j].d_scale) return DQ_ERR_NOT_SUPPORTED;
        hj[j] = {DQ_FMT_Q8_0, jobs[j].d_qs, jobs[j].rows, jobs[j].y};
    }
    return run_host_jobs(hj.data(), n, cols, x);
}

int matmul_q8_0_cuda(const uint8_t* q8_data, size_t rows, size_t cols, const float* x, float* y) {
    if (!q8_data || !gemv_shape_ok(DQ_FMT_Q8_0, rows, cols)) return DQ_ERR_NOT_SUPPORTED;
    if (!x || !y) return DQ_ERR_INVALID_ARG;
    if (!stream()) return DQ_ERR_IO;
    DqLayout L;
    dq_layout(DQ_FMT_Q8_0, rows, cols, &L);
    const size_t gguf = rows * dq_gguf_row_bytes(DQ_FMT_Q8_0, cols);
    if (!reserve(g.work, L.total) || !reserve(g.stage, gguf)) return DQ_ERR_IO;
    if (hipMemcpyAsync(g.stage.p, q8_data, gguf, hipMemcpyHostToDevice, g.stream) != hipSuccess) return io_fail();
    if (dq_weights_pack(DQ_FMT_Q8_0, g.stage.p, rows, cols, g.work.p, g.stream) != DQ_OK) return io_fail();
    const HostJob j = {DQ_FMT_Q8_0, g.work.p, rows, y};
    return run_host_jobs(&j, 1, cols, x);
}

int matmul_kquant_cuda_batch(int format, const void* d_w, size_t rows, size_t cols, const float* x, size_t n_tok,
                             float* y) {
    if (format != DQ_FMT_Q4_K && format != DQ_FMT_Q6_K && format != DQ_FMT_Q8_0 && format != DQ_FMT_Q4_0)
        return DQ_ERR_NOT_SUPPORTED;
    if (!d_w || rows == 0 || n_tok == 0 || cols == 0 || cols % 256 || !gemv_shape_ok(format, rows, cols))
        return DQ_ERR_NOT_SUPPORTED;
    if (rows > (1u << 30) || n_tok > (1u << 20)) return DQ_ERR_NOT_SUPPORTED;
    if (!x || !y) return DQ_ERR_INVALID_ARG;
    // matmul_<fmt>_batch take the i8_gemm path from 4 tokens (Q8_0: from 2,
    // core/matmul.cpp:848-860, 2090-2125)
    if (n_tok < (format == DQ_FMT_Q8_0 ? 2u : 4u)) {
        // below the i8_gemm threshold: the single-column GEMV per token
        for (size_t t = 0; t < n_tok; ++t) {
            const HostJob j = {format, d_w, rows, y + t * rows};
            const int rc = run_host_jobs(&j, 1, cols, x + t * cols);
            if (rc != DQ_OK) return rc;
        }
        return DQ_OK;
    }
    size_t wbytes = 0;
    if (dq_gemm_workspace_bytes(format, rows, cols, n_tok, &wbytes) != DQ_OK) return DQ_ERR_NOT_SUPPORTED;
    if (!stream()) return DQ_ERR_IO;
    if (!reserve(g.xbuf, n_tok * cols * 4) || !reserve(g.ybuf, n_tok * rows * 4) || !reserve(g.work, wbytes))
        return DQ_ERR_IO;
    if (hipMemcpyAsync(g.xbuf.p, x, n_tok * cols * 4, hipMemcpyHostToDevice, g.stream) != hipSuccess) return io_fail();
    // the matrix's tile copy where the engine keeps one (same results)
    const WInfo* wi = lookup(d_w);
    const bool tl = wi && wi->base == d_w && wi->tiles;
    const int rc = dq_gemm(tl ? (format | DQ_FMT_GEMM_TILES) : format, tl ? wi->tiles : d_w, rows, cols,
                           (const float*)g.xbuf.p, n_tok, (float*)g.ybuf.p, g.work.p, g.work.cap, g.stream);
    if (rc != DQ_OK) return rc == DQ_ERR_IO ? io_fail() : rc;
    if (hipMemcpyAsync(y, g.ybuf.p, n_tok * rows * 4, hipMemcpyDeviceToHost, g.stream) != hipSuccess) return io_fail();
    return sync();
}

int matmul_q8_0_cuda_ffn_gated(const void* d_up_qs, const void* d_up_scale, const void* d_gate_qs,
                               const void* d_gate_scale, const void* d_down_qs, const void* d_down_scale, size_t n_ff,
                               size_t n_embd, const float* x, float* out, int act_gelu) {
    if (!d_up_qs || !d_up_scale || !d_gate_qs || !d_gate_scale || !d_down_qs || !d_down_scale)
        return DQ_ERR_NOT_SUPPORTED;
    if (!gemv_shape_ok(DQ_FMT_Q8_0, n_ff, n_embd) || !gemv_shape_ok(DQ_FMT_Q8_0, n_embd, n_ff))
        return DQ_ERR_NOT_SUPPORTED;
    if (!x || !out) return DQ_ERR_INVALID_ARG;
    if (!stream()) return DQ_ERR_IO;
    const size_t mx = n_ff > n_embd ? n_ff : n_embd;
    if (!reserve(g.xbuf, mx * 4) || !reserve(g.act, act_bytes(mx)) || !reserve(g.ybuf, (3 * n_ff + n_embd) * 4))
        return DQ_ERR_IO;
    const hipStream_t s = g.stream;
    float* dx = (float*)g.xbuf.p;
    float* up = (float*)g.ybuf.p;
    float* gate = up + n_ff;
    float* h = gate + n_ff;
    float* dout = h + n_ff;
    const Act a = carve_act((uint8_t*)g.act.p, mx);
    if (hipMemcpyAsync(dx, x, n_embd * 4, hipMemcpyHostToDevice, s) != hipSuccess) return io_fail();
    // matvec(up), matvec(gate) (matmul_q8_0: per-32 quantization of x),
    // silu(gate) * up or geglu (the decode branch, dense_forward.cpp
    // :4212-4219), matvec(down) (per-32 quantization of h)
    const dq_gemv_job_t jobs[2] = {{DQ_FMT_Q8_0, d_up_qs, n_ff, up, nullptr}, {DQ_FMT_Q8_0, d_gate_qs, n_ff, gate, nullptr}};
    if (dq_quantize_act(DQ_ACT_Q8_0, dx, n_embd, 1, a.q, a.s, a.i, nullptr, s) != DQ_OK ||
        dq_gemv_group(jobs, 2, n_embd, a.q, a.s, a.i, s) != DQ_OK || dq_act_mul(gate, up, n_ff, act_gelu ? 1 : 0, h, s) != DQ_OK ||
        dq_quantize_act(DQ_ACT_Q8_0, h, n_ff, 1, a.q, a.s, a.i, nullptr, s) != DQ_OK ||
        dq_gemv(DQ_FMT_Q8_0, d_down_qs, n_embd, n_ff, a.q, a.s, a.i, dout, s) != DQ_OK)
        return io_fail();
    if (hipMemcpyAsync(out, dout, n_embd * 4, hipMemcpyDeviceToHost, s) != hipSuccess) return io_fail();
    return sync();
}

// --------------------------------------------------------------- KV cache --

bool cuda_kv_cache_reserve(size_t total_bytes) {
    if (total_bytes <= g.kv_bytes && g.kc) return true;
    // graphs hold the cache addresses: a new cache invalidates them
    if (g.stream) (void)hipStreamSynchronize(g.stream);
    drop_graphs();
    if (g.kc) (void)hipFree(g.kc);
    if (g.vc) (void)hipFree(g.vc);
    g.kc = g.vc = nullptr;
    g.kv_bytes = 0;
    if (total_bytes == 0) return true;
    if (hipMalloc((void**)&g.kc, total_bytes) != hipSuccess) {
        (void)hipGetLastError();
        g.kc = nullptr;
        return false;
    }
    if (hipMalloc((void**)&g.vc, total_bytes) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(g.kc);
        g.kc = nullptr;
        return false;
    }
    g.kv_bytes = total_bytes;
    return true;
}

void cuda_kv_cache_release(void) {
    if (g.stream) (void)hipStreamSynchronize(g.stream);
    drop_graphs();
    if (g.kc) (void)hipFree(g.kc);
    if (g.vc) (void)hipFree(g.vc);
    g.kc = g.vc = nullptr;
    g.kv_bytes = 0;
}

bool cuda_kv_cache_upload(const void* k_host, const void* v_host, size_t total_bytes) {
    if (!g.kc || total_bytes > g.kv_bytes || !k_host || !v_host || !stream()) return false;
    const bool ok = hipMemcpyAsync(g.kc, k_host, total_bytes, hipMemcpyHostToDevice, g.stream) == hipSuccess &&
                    hipMemcpyAsync(g.vc, v_host, total_bytes, hipMemcpyHostToDevice, g.stream) == hipSuccess &&
                    hipStreamSynchronize(g.stream) == hipSuccess;
    if (!ok) (void)hipGetLastError();
    return ok;
}

bool cuda_kv_cache_download(void* k_host, void* v_host, size_t total_bytes) {
    if (!g.kc || total_bytes > g.kv_bytes || !k_host || !v_host || !stream()) return false;
    const bool ok = hipMemcpyAsync(k_host, g.kc, total_bytes, hipMemcpyDeviceToHost, g.stream) == hipSuccess &&
                    hipMemcpyAsync(v_host, g.vc, total_bytes, hipMemcpyDeviceToHost, g.stream) == hipSuccess &&
                    hipStreamSynchronize(g.stream) == hipSuccess;
    if (!ok) (void)hipGetLastError();
    return ok;
}

bool cuda_kv_cache_write(size_t byte_off, const void* k, const void* v, size_t bytes) {
    if (!g.kc || byte_off > g.kv_bytes || bytes > g.kv_bytes - byte_off || !k || !v || !stream()) return false;
    // pageable sources: the copies have read them when the calls return
    const bool ok = hipMemcpyAsync(g.kc + byte_off, k, bytes, hipMemcpyHostToDevice, g.stream) == hipSuccess &&
                    hipMemcpyAsync(g.vc + byte_off, v, bytes, hipMemcpyHostToDevice, g.stream) == hipSuccess;
    if (!ok) (void)hipGetLastError();
    return ok;
}

bool cuda_kv_cache_read(size_t byte_off, void* k, void* v, size_t bytes) {
    if (!g.kc || byte_off > g.kv_bytes || bytes > g.kv_bytes - byte_off || !k || !v || !stream()) return false;
    const bool ok = hipMemcpyAsync(k, g.kc + byte_off, bytes, hipMemcpyDeviceToHost, g.stream) == hipSuccess &&
                    hipMemcpyAsync(v, g.vc + byte_off, bytes, hipMemcpyDeviceToHost, g.stream) == hipSuccess &&
                    hipStreamSynchronize(g.stream) == hipSuccess;
    if (!ok) (void)hipGetLastError();
    return ok;
}

bool cuda_kv_cache_move(size_t dst_off, size_t src_off, size_t bytes) {
    if (bytes == 0 || dst_off == src_off) return true;
    const size_t hi = dst_off > src_off ? dst_off : src_off;
    if (!g.kc || hi > g.kv_bytes || bytes > g.kv_bytes - hi || !stream()) return false;
    // the ranges may overlap: through the staging buffer, K then V
    if (!reserve(g.stage, bytes)) return false;
    bool ok = true;
    for (uint8_t* base : {g.kc, g.vc}) {
        ok = ok && hipMemcpyAsync(g.stage.p, base + src_off, bytes, hipMemcpyDeviceToDevice, g.stream) == hipSuccess &&
             hipMemcpyAsync(base + dst_off, g.stage.p, bytes, hipMemcpyDeviceToDevice, g.stream) == hipSuccess;
    }
    ok = ok && hipStreamSynchronize(g.stream) == hipSuccess;
    if (!ok) (void)hipGetLastError();
    return ok;
}

void cuda_set_attention_long(bool long_context) {
    // One decode-attention kernel covers every context length here (split
    // over positions when the context is long); nothing to switch.
    (void)long_context;
}

void cuda_drop_graphs(void) {
    if (g.stream) (void)hipStreamSynchronize(g.stream);
    drop_graphs();
}

// -------------------------------------------------------------- attention --

int cuda_attention_out(const void* d_wo_qs, const void* d_wo_scale, const float* q, uint32_t n_head,
                       uint32_t heads_per_kv, uint32_t head_dim, uint32_t kv_dim, size_t layer_off, uint32_t cc_start,
                       uint32_t pos, size_t n_embd, size_t q_dim, float* proj, int kv_quantized, size_t row_bytes) {
    if (!g.kc || !d_wo_qs || !d_wo_scale || !kv_quantized) return DQ_ERR_NOT_SUPPORTED;
    const WInfo* wo = lookup(d_wo_qs);
    if (!wo || wo->rows != n_embd || wo->cols != q_dim) return DQ_ERR_NOT_SUPPORTED;
    if (heads_per_kv == 0 || n_head % heads_per_kv || !dq_head_dim_supported(head_dim)) return DQ_ERR_NOT_SUPPORTED;
    const uint32_t n_kv = n_head / heads_per_kv;
    if ((size_t)n_head * head_dim != q_dim || (size_t)n_kv * head_dim != kv_dim) return DQ_ERR_NOT_SUPPORTED;
    if (row_bytes != (size_t)(head_dim / 32) * DQ_SZ_Q8_0) return DQ_ERR_NOT_SUPPORTED;
    const size_t pb = kv_pos_bytes(n_kv, head_dim);
    const uint32_t n_ctx = kv_positions(layer_off, pb);
    if (pos >= n_ctx || cc_start > pos) return DQ_ERR_NOT_SUPPORTED;
    if (!gemv_shape_ok(wo->fmt, n_embd, q_dim)) return DQ_ERR_NOT_SUPPORTED;
    size_t ab = 0;
    if (dq_attn_workspace_bytes(n_head, n_kv, head_dim, n_ctx, &ab) != DQ_OK) return DQ_ERR_NOT_SUPPORTED;
    if (!q || !proj) return DQ_ERR_INVALID_ARG;
    if (!stream()) return DQ_ERR_IO;
    if (!reserve(g.xbuf, 2 * q_dim * 4) || !reserve(g.act, act_bytes(q_dim)) || !reserve(g.ybuf, n_embd * 4) ||
        !reserve(g.work, ab))
        return DQ_ERR_IO;
    const hipStream_t s = g.stream;
    float* dq = (float*)g.xbuf.p;
    float* dao = dq + q_dim;
    const Act a = carve_act((uint8_t*)g.act.p, q_dim);
    if (hipMemcpyAsync(dq, q, q_dim * 4, hipMemcpyHostToDevice, s) != hipSuccess) return io_fail();
    if (dq_attn_decode_q8(dq, g.kc + layer_off, g.vc + layer_off, n_head, n_kv, head_dim, cc_start, pos, nullptr, n_ctx,
                          dao, g.work.p, g.work.cap, s) != DQ_OK ||
        dq_quantize_act(act_kind(wo->fmt), dao, q_dim, 1, a.q, a.s, a.i, nullptr, s) != DQ_OK ||
        dq_gemv(wo->fmt, d_wo_qs, n_embd, q_dim, a.q, a.s, a.i, (float*)g.ybuf.p, s) != DQ_OK)
        return io_fail();
    if (hipMemcpyAsync(proj, g.ybuf.p, n_embd * 4, hipMemcpyDeviceToHost, s) != hipSuccess) return io_fail();
    return sync();
}

int cuda_qkv_attention_out(const CudaQkvAttnArgs* A) {
    if (!A || !g.kc) return DQ_ERR_NOT_SUPPORTED;
    const WInfo* m[4] = {lookup(A->wq_qs), lookup(A->wk_qs), lookup(A->wv_qs), lookup(A->wo_qs)};
    for (const WInfo* w : m)
        if (!w) return DQ_ERR_NOT_SUPPORTED;
    if (!dq_head_dim_supported(A->head_dim) || A->n_head_kv == 0 || A->n_head % A->n_head_kv) return DQ_ERR_NOT_SUPPORTED;
    if (A->heads_per_kv != A->n_head / A->n_head_kv) return DQ_ERR_NOT_SUPPORTED;
    const size_t E = A->n_embd, QD = A->q_dim, KVD = A->kv_dim;
    if (QD != (size_t)A->n_head * A->head_dim || KVD != (size_t)A->n_head_kv * A->head_dim) return DQ_ERR_NOT_SUPPORTED;
    if (m[0]->rows != QD || m[1]->rows != KVD || m[2]->rows != KVD || m[3]->rows != E) return DQ_ERR_NOT_SUPPORTED;
    if (m[0]->cols != E || m[1]->cols != E || m[2]->cols != E || m[3]->cols != QD) return DQ_ERR_NOT_SUPPORTED;
    for (int j = 0; j < 4; ++j)
        if (!gemv_shape_ok(m[j]->fmt, m[j]->rows, m[j]->cols) ||
            (act_kind(m[j]->fmt) == DQ_ACT_Q8K_REP && m[j]->cols % 256))
            return DQ_ERR_NOT_SUPPORTED;
    if (A->rope_cache && (A->n_rot == 0 || A->n_rot > A->head_dim || A->n_rot % 2)) return DQ_ERR_NOT_SUPPORTED;
    const size_t pb = kv_pos_bytes(A->n_head_kv, A->head_dim);
    const uint32_t n_ctx = kv_positions(A->kv_layer_off, pb);
    if (A->pos >= n_ctx || A->cc_start > A->pos) return DQ_ERR_NOT_SUPPORTED;
    size_t ab = 0;
    if (dq_attn_workspace_bytes(A->n_head, A->n_head_kv, A->head_dim, n_ctx, &ab) != DQ_OK) return DQ_ERR_NOT_SUPPORTED;
    if (!A->attn_in || !A->proj) return DQ_ERR_INVALID_ARG;
    if (!stream()) return DQ_ERR_IO;
    const size_t mx = E > QD ? E : QD;
    // x, q, k, v, attention out, proj, biases
    const size_t nf = E + QD + 2 * KVD + QD + E + QD + 2 * KVD;
    if (!reserve(g.xbuf, nf * 4) || !reserve(g.act, 2 * act_bytes(mx)) || !reserve(g.work, ab) ||
        !reserve(g.rope, 512 * 4))
        return DQ_ERR_IO;
    const hipStream_t s = g.stream;
    float* dx = (float*)g.xbuf.p;
    float* dq = dx + E;
    float* dk = dq + QD;
    float* dv = dk + KVD;
    float* dao = dv + KVD;
    float* dproj = dao + QD;
    float* db[3] = {dproj + E, dproj + E + QD, dproj + E + QD + KVD};
    const float* hb[3] = {A->bq, A->bk, A->bv};
    const size_t bn[3] = {QD, KVD, KVD};
    Act a[2] = {carve_act((uint8_t*)g.act.p, mx), carve_act((uint8_t*)g.act.p + act_bytes(mx), mx)};
    if (hipMemcpyAsync(dx, A->attn_in, E * 4, hipMemcpyHostToDevice, s) != hipSuccess) return io_fail();
    for (int j = 0; j < 3; ++j)
        if (hb[j] && hipMemcpyAsync(db[j], hb[j], bn[j] * 4, hipMemcpyHostToDevice, s) != hipSuccess) return io_fail();
    if (A->rope_cache &&
        hipMemcpyAsync(g.rope.p, A->rope_cache, (size_t)A->n_rot * 4, hipMemcpyHostToDevice, s) != hipSuccess)
        return io_fail();
    // Q/K/V, each on the activation its format's reference GEMV uses; the
    // bias is added to the GEMV result (the residual slot of the epilogue)
    bool need[2] = {false, false};
    for (int j = 0; j < 3; ++j) need[act_kind(m[j]->fmt)] = true;
    for (int k = 0; k < 2; ++k)
        if (need[k] && dq_quantize_act(k, dx, E, 1, a[k].q, a[k].s, a[k].i, nullptr, s) != DQ_OK) return io_fail();
    const void* wp[3] = {A->wq_qs, A->wk_qs, A->wv_qs};
    float* yp[3] = {dq, dk, dv};
    for (int k = 0; k < 2; ++k) {
        dq_gemv_job_t jobs[3];
        int n = 0;
        for (int j = 0; j < 3; ++j)
            if (act_kind(m[j]->fmt) == k) jobs[n++] = {m[j]->fmt, wp[j], m[j]->rows, yp[j], hb[j] ? db[j] : nullptr};
        if (n && dq_gemv_group(jobs, (size_t)n, E, a[k].q, a[k].s, a[k].i, s) != DQ_OK) return io_fail();
    }
    uint8_t* kc = g.kc + A->kv_layer_off;
    uint8_t* vc = g.vc + A->kv_layer_off;
    const int kwo = act_kind(m[3]->fmt);
    if (dq_rope_kv_write(dq, dk, dv, A->rope_cache ? (const float*)g.rope.p : nullptr, A->n_head, A->n_head_kv,
                         A->head_dim, A->n_rot, kc, vc, A->pos, nullptr, n_ctx, s) != DQ_OK ||
        dq_attn_decode_q8(dq, kc, vc, A->n_head, A->n_head_kv, A->head_dim, A->cc_start, A->pos, nullptr, n_ctx, dao,
                          g.work.p, g.work.cap, s) != DQ_OK ||
        dq_quantize_act(kwo, dao, QD, 1, a[kwo].q, a[kwo].s, a[kwo].i, nullptr, s) != DQ_OK ||
        dq_gemv(m[3]->fmt, A->wo_qs, E, QD, a[kwo].q, a[kwo].s, a[kwo].i, dproj, s) != DQ_OK)
        return io_fail();
    // the host cache slot of this position follows the device copy
    const size_t row_off = (size_t)A->pos * pb;
    if (A->host_k_row && hipMemcpyAsync(A->host_k_row, kc + row_off, pb, hipMemcpyDeviceToHost, s) != hipSuccess)
        return io_fail();
    if (A->host_v_row && hipMemcpyAsync(A->host_v_row, vc + row_off, pb, hipMemcpyDeviceToHost, s) != hipSuccess)
        return io_fail();
    if (hipMemcpyAsync(A->proj, dproj, E * 4, hipMemcpyDeviceToHost, s) != hipSuccess) return io_fail();
    return sync();
}

// ------------------------------------------------------------------ layer --

// The optional per-layer vectors (Q/K/V biases, QK-norm weights, sandwich
// norms): host pointers (NULL = absent) and float counts.
struct LayerExtras {
    static constexpr int N = 7;
    const float* h[N];
    size_t n[N];
    size_t bytes() const {
        size_t b = 0;
        for (int i = 0; i < N; ++i)
            if (h[i]) b += dq_align256(n[i] * 4);
        return b;
    }
    // device copies at dst (each 256-byte aligned), pointers into the layer
    bool upload(dq_layer_t& L, uint8_t* dst, hipStream_t s) const {
        const float** d[N] = {&L.bq, &L.bk, &L.bv, &L.q_norm, &L.k_norm, &L.post_attn_norm, &L.post_ffn_norm};
        for (int i = 0; i < N; ++i) {
            *d[i] = nullptr;
            if (!h[i]) continue;
            if (hipMemcpyAsync(dst, h[i], n[i] * 4, hipMemcpyHostToDevice, s) != hipSuccess) return false;
            *d[i] = (const float*)dst;
            dst += dq_align256(n[i] * 4);
        }
        return true;
    }
};
static LayerExtras extras_of(const float* bq, const float* bk, const float* bv, const float* qn, const float* kn,
                             const float* pa, const float* pf, size_t q_dim, size_t kv_dim, size_t hd, size_t E) {
    return LayerExtras{{bq, bk, bv, qn, kn, pa, pf}, {q_dim, kv_dim, kv_dim, hd, hd, E, E}};
}

int cuda_layer_forward(const CudaLayerArgs* A) {
    if (!A || !g.kc) return DQ_ERR_NOT_SUPPORTED;
    if (!A->attn_norm_w || !A->ffn_norm_w) return DQ_ERR_NOT_SUPPORTED;
    // per-layer slots (models whose layers differ in window or RoPE base,
    // dense_forward.cpp:3760-3788): the (pos, cc_start) pairs [n_slots][2]
    // and RoPE tables [n_slots][rope_stride] of every layer; this layer reads
    // slot layer_slot (backend_cuda.cu:4330-4366). The tables go to the
    // device with the first layer of a token (upload_x); the pair is read
    // from the host array every layer passes.
    const bool slots = A->dyn_all && A->layer_slot < A->n_slots;
    if (slots && A->rope_cache && (!A->rope_all || A->rope_stride < A->n_rot)) return DQ_ERR_INVALID_ARG;
    const uint32_t pos = slots ? A->dyn_all[2 * (size_t)A->layer_slot] : A->pos;
    const uint32_t cc_start = slots ? A->dyn_all[2 * (size_t)A->layer_slot + 1] : A->cc_start;
    if (!dq_head_dim_supported(A->head_dim) || A->n_head_kv == 0 || A->n_head % A->n_head_kv ||
        A->heads_per_kv != A->n_head / A->n_head_kv)
        return DQ_ERR_NOT_SUPPORTED;
    if (A->q_dim != (size_t)A->n_head * A->head_dim || A->kv_dim != (size_t)A->n_head_kv * A->head_dim)
        return DQ_ERR_NOT_SUPPORTED;
    if (A->n_embd > 0xFFFFFFFFu || A->n_ff > 0xFFFFFFFFu) return DQ_ERR_NOT_SUPPORTED;
    if (A->rope_cache && (A->n_rot == 0 || A->n_rot > A->head_dim || A->n_rot % 2)) return DQ_ERR_NOT_SUPPORTED;
    dq_layer_t L{};
    L.n_embd = (uint32_t)A->n_embd;
    L.n_head = A->n_head;
    L.n_head_kv = A->n_head_kv;
    L.head_dim = A->head_dim;
    L.n_rot = A->rope_cache ? A->n_rot : A->head_dim;
    L.n_ff = (uint32_t)A->n_ff;
    L.rms_eps = A->rms_eps;
    L.act_gelu = A->act_gelu ? 1 : 0;
    L.fmt_q = A->fmt_q, L.fmt_k = A->fmt_k, L.fmt_v = A->fmt_v, L.fmt_o = A->fmt_o;
    L.fmt_gate = A->fmt_gate, L.fmt_up = A->fmt_up, L.fmt_down = A->fmt_down;
    L.wq = A->wq_qs, L.wk = A->wk_qs, L.wv = A->wv_qs, L.wo = A->wo_qs;
    L.wgate = A->wgate_qs, L.wup = A->wup_qs, L.wdown = A->wdown_qs;
    L.attn_norm = A->attn_norm_w;  // host pointers here; device copies below
    L.ffn_norm = A->ffn_norm_w;
    L.post_attn_norm = A->post_attn_norm_w;  // (their presence sizes the workspace)
    L.post_ffn_norm = A->post_ffn_norm_w;
    L.wag = A->wag_qs, L.fmt_ag = A->fmt_ag;  // optional per-head attention output gate
    // every matrix must be one of ours, of the declared format and shape
    const void* w[8] = {L.wq, L.wk, L.wv, L.wo, L.wgate, L.wup, L.wdown, L.wag};
    const int f[8] = {L.fmt_q, L.fmt_k, L.fmt_v, L.fmt_o, L.fmt_gate, L.fmt_up, L.fmt_down, L.fmt_ag};
    const size_t r[8] = {A->q_dim, A->kv_dim, A->kv_dim, A->n_embd, A->n_ff, A->n_ff, A->n_embd, A->n_head};
    const size_t c[8] = {A->n_embd, A->n_embd, A->n_embd, A->q_dim, A->n_embd, A->n_embd, A->n_ff, A->n_embd};
    for (int j = 0; j < (L.wag ? 8 : 7); ++j) {
        const WInfo* wi = lookup(w[j]);
        if (!wi || wi->base != w[j] || wi->fmt != f[j] || wi->rows != r[j] || wi->cols != c[j])
            return DQ_ERR_NOT_SUPPORTED;
    }
    const size_t pb = kv_pos_bytes(A->n_head_kv, A->head_dim);
    const uint32_t n_ctx = kv_positions(A->kv_layer_off, pb);
    if (pos >= n_ctx || cc_start > pos) return DQ_ERR_NOT_SUPPORTED;
    size_t wbytes = 0;
    if (dq_layer_workspace_bytes(&L, n_ctx, &wbytes) != DQ_OK) return DQ_ERR_NOT_SUPPORTED;
    // x_from_token: x is the Q8_0 embedding row of the token the previous
    // step drew on the device (pipelined decode)
    const WInfo* emb = nullptr;
    if (A->x_from_token) {
        emb = lookup(A->embd_qs);
        if (!A->upload_x || !emb || emb->base != A->embd_qs || emb->fmt != DQ_FMT_Q8_0 || emb->cols != A->n_embd ||
            !g.sst)
            return DQ_ERR_NOT_SUPPORTED;
    }
    if (A->upload_x && !A->x && !A->x_from_token) return DQ_ERR_INVALID_ARG;
    if (A->download_x && !A->x_out) return DQ_ERR_INVALID_ARG;
    if (!stream()) return DQ_ERR_IO;
    const size_t E = A->n_embd;
    // norm weights and the optional biases / QK-norm weights: device copies in
    // the tail of the workspace
    const LayerExtras ex =
        extras_of(A->bq, A->bk, A->bv, A->q_norm_w, A->k_norm_w, A->post_attn_norm_w, A->post_ffn_norm_w, A->q_dim,
                  A->kv_dim, A->head_dim, A->n_embd);
    const size_t norm_off = dq_align256(wbytes);
    if (!reserve(g.work, norm_off + 2 * dq_align256(E * 4) + ex.bytes()) || !reserve(g.lx[0], E * 4) ||
        !reserve(g.lx[1], E * 4))
        return DQ_ERR_IO;
    const hipStream_t s = g.stream;
    float* an = (float*)((uint8_t*)g.work.p + norm_off);
    float* fn = (float*)((uint8_t*)g.work.p + norm_off + dq_align256(E * 4));
    if (hipMemcpyAsync(an, A->attn_norm_w, E * 4, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipMemcpyAsync(fn, A->ffn_norm_w, E * 4, hipMemcpyHostToDevice, s) != hipSuccess ||
        !ex.upload(L, (uint8_t*)g.work.p + norm_off + 2 * dq_align256(E * 4), s))
        return io_fail();
    L.attn_norm = an;
    L.ffn_norm = fn;
    const float* d_rope = nullptr;
    if (slots) {
        // Every slot's table goes to the device with the token's first layer
        // (upload_x), whether or not that layer rotates: a first layer without
        // RoPE must not leave the later layers on the previous token's tables
        // (backend_cuda.cu:4331-4345).
        const size_t nr = (size_t)A->n_slots * A->rope_stride;
        if (A->rope_all && nr && (A->upload_x || g.rope_all_n != nr)) {
            g.rope_all_n = 0;
            if (!reserve(g.rope_all, nr * 4)) return DQ_ERR_IO;
            if (hipMemcpyAsync(g.rope_all.p, A->rope_all, nr * 4, hipMemcpyHostToDevice, s) != hipSuccess)
                return io_fail();
            g.rope_all_n = nr;
        }
        if (A->rope_cache) d_rope = (const float*)g.rope_all.p + (size_t)A->layer_slot * A->rope_stride;
    } else {
        if (A->upload_dyn || !g.rope.p) {
            const int rc = upload_rope(A->rope_cache, A->n_rot);
            if (rc != DQ_OK) return rc;
        }
        d_rope = g.rope_on ? (const float*)g.rope.p : nullptr;
    }
    if (A->upload_x) {
        g.cur = 0;
        if (A->x_from_token) {
            if (dq_embed_q8_0(A->embd_qs, emb->rows, E, &g.sst->tok, A->embd_mul, (float*)g.lx[0].p, s) != DQ_OK)
                return io_fail();
        } else if (hipMemcpyAsync(g.lx[0].p, A->x, E * 4, hipMemcpyHostToDevice, s) != hipSuccess) {
            return io_fail();
        }
    }
    float* xin = (float*)g.lx[g.cur].p;
    float* xout = (float*)g.lx[g.cur ^ 1].p;
    const int rc = dq_layer_decode(&L, xin, xout, d_rope, pos, nullptr, cc_start, g.kc + A->kv_layer_off,
                                   g.vc + A->kv_layer_off, n_ctx, g.work.p, norm_off, s);
    if (rc != DQ_OK) return rc == DQ_ERR_IO ? io_fail() : rc;
    g.cur ^= 1;
    if (A->download_x) {
        if (hipMemcpyAsync(A->x_out, xout, E * 4, hipMemcpyDeviceToHost, s) != hipSuccess) return io_fail();
        return sync();
    }
    return DQ_OK;
}

int cuda_attention_batch(const float* q_all, float* out_all, uint32_t n_tokens, uint32_t n_head,
                         uint32_t heads_per_kv, uint32_t head_dim, uint32_t q_dim, size_t row_bytes, size_t pos_bytes,
                         size_t layer_off, uint32_t col0, uint32_t n_swa) {
    if (!g.kc || n_tokens == 0 || n_head == 0 || heads_per_kv == 0 || n_head % heads_per_kv)
        return DQ_ERR_NOT_SUPPORTED;
    if (head_dim != 64 && head_dim != 128 && head_dim != 256) return DQ_ERR_NOT_SUPPORTED;
    const uint32_t n_kv = n_head / heads_per_kv;
    if (row_bytes != (size_t)(head_dim / 32) * DQ_SZ_Q8_0 || pos_bytes != kv_pos_bytes(n_kv, head_dim))
        return DQ_ERR_NOT_SUPPORTED;
    if ((size_t)q_dim < (size_t)n_head * head_dim || q_dim % 4 || layer_off % 4) return DQ_ERR_NOT_SUPPORTED;
    const uint32_t n_ctx = kv_positions(layer_off, pos_bytes);
    if ((uint64_t)col0 + n_tokens > n_ctx) return DQ_ERR_NOT_SUPPORTED;
    if (!q_all || !out_all) return DQ_ERR_INVALID_ARG;
    if (!stream()) return DQ_ERR_IO;
    const size_t n = (size_t)n_tokens * q_dim;
    size_t ab = 0;
    if (dq_attn_prefill_workspace_bytes(n_tokens, n_head, n_kv, head_dim, &ab) != DQ_OK) return DQ_ERR_NOT_SUPPORTED;
    if (!reserve(g.pio, 2 * dq_align256(n * 4) + ab)) return DQ_ERR_IO;
    const hipStream_t s = g.stream;
    float* dq = (float*)g.pio.p;
    float* dout = (float*)((uint8_t*)g.pio.p + dq_align256(n * 4));
    void* dwork = (uint8_t*)g.pio.p + 2 * dq_align256(n * 4);
    if (hipMemcpyAsync(dq, q_all, n * 4, hipMemcpyHostToDevice, s) != hipSuccess) return io_fail();
    // columns past the heads keep the caller's values
    if ((size_t)q_dim > (size_t)n_head * head_dim &&
        hipMemcpyAsync(dout, out_all, n * 4, hipMemcpyHostToDevice, s) != hipSuccess)
        return io_fail();
    if (dq_attn_prefill_q8(dq, g.kc + layer_off, g.vc + layer_off, n_tokens, n_head, n_kv, head_dim, q_dim, col0,
                           n_swa, n_ctx, dout, dwork, ab, s) != DQ_OK)
        return io_fail();
    if (hipMemcpyAsync(out_all, dout, n * 4, hipMemcpyDeviceToHost, s) != hipSuccess) return io_fail();
    return sync();
}

int cuda_layer_forward_batch(const struct CudaLayerBatchArgs* A) {
    if (!A || !g.kc || A->n_tok == 0 || A->n_total == 0) return DQ_ERR_NOT_SUPPORTED;
    if (!A->attn_norm_w || !A->ffn_norm_w) return DQ_ERR_NOT_SUPPORTED;
    if (!dq_head_dim_supported(A->head_dim) || A->n_head_kv == 0 || A->n_head % A->n_head_kv ||
        A->heads_per_kv != A->n_head / A->n_head_kv)
        return DQ_ERR_NOT_SUPPORTED;
    if (A->q_dim != (size_t)A->n_head * A->head_dim || A->kv_dim != (size_t)A->n_head_kv * A->head_dim)
        return DQ_ERR_NOT_SUPPORTED;
    if (A->n_embd > 0xFFFFFFFFu || A->n_ff > 0xFFFFFFFFu) return DQ_ERR_NOT_SUPPORTED;
    if ((uint64_t)A->x_row0 + A->n_tok > A->n_total || A->n_tok > 65535) return DQ_ERR_NOT_SUPPORTED;
    if (A->rope_caches && (A->n_rot == 0 || A->n_rot > A->head_dim || A->n_rot % 2 || A->rope_slot < 0 ||
                           A->rope_slot > 3))
        return DQ_ERR_NOT_SUPPORTED;
    dq_layer_t L{};
    L.n_embd = (uint32_t)A->n_embd;
    L.n_head = A->n_head;
    L.n_head_kv = A->n_head_kv;
    L.head_dim = A->head_dim;
    L.n_rot = A->rope_caches ? A->n_rot : A->head_dim;
    L.n_ff = (uint32_t)A->n_ff;
    L.rms_eps = A->rms_eps;
    L.act_gelu = A->act_gelu ? 1 : 0;
    L.fmt_q = A->fmt_q, L.fmt_k = A->fmt_k, L.fmt_v = A->fmt_v, L.fmt_o = A->fmt_o;
    L.fmt_gate = A->fmt_gate, L.fmt_up = A->fmt_up, L.fmt_down = A->fmt_down;
    L.wq = A->wq_qs, L.wk = A->wk_qs, L.wv = A->wv_qs, L.wo = A->wo_qs;
    L.wgate = A->wgate_qs, L.wup = A->wup_qs, L.wdown = A->wdown_qs;
    L.wag = A->wag_qs, L.fmt_ag = A->fmt_ag;  // optional per-head attention output gate
    const void* w[8] = {L.wq, L.wk, L.wv, L.wo, L.wgate, L.wup, L.wdown, L.wag};
    const int f[8] = {L.fmt_q, L.fmt_k, L.fmt_v, L.fmt_o, L.fmt_gate, L.fmt_up, L.fmt_down, L.fmt_ag};
    const size_t r[8] = {A->q_dim, A->kv_dim, A->kv_dim, A->n_embd, A->n_ff, A->n_ff, A->n_embd, A->n_head};
    const size_t c[8] = {A->n_embd, A->n_embd, A->n_embd, A->q_dim, A->n_embd, A->n_embd, A->n_ff, A->n_embd};
    const void** tl[8] = {&L.tq, &L.tk, &L.tv, &L.to, &L.tgate, &L.tup, &L.tdown, &L.tag};
    for (int j = 0; j < (L.wag ? 8 : 7); ++j) {
        const WInfo* wi = lookup(w[j]);
        if (!wi || wi->base != w[j] || wi->fmt != f[j] || wi->rows != r[j] || wi->cols != c[j])
            return DQ_ERR_NOT_SUPPORTED;
        *tl[j] = wi->tiles;  // the products read the tile copies where they exist
    }
    size_t wbytes = 0;
    if (dq_layer_prefill_workspace_bytes(&L, A->n_tok, &wbytes) != DQ_OK) return DQ_ERR_NOT_SUPPORTED;
    const size_t pb = kv_pos_bytes(A->n_head_kv, A->head_dim);
    const uint32_t n_ctx = kv_positions(A->kv_layer_off, pb);
    if ((uint64_t)A->pos0 + A->n_tok > n_ctx) return DQ_ERR_NOT_SUPPORTED;
    if (A->upload_x && !A->x) return DQ_ERR_INVALID_ARG;
    if (A->download_x && !A->x_out) return DQ_ERR_INVALID_ARG;
    if (A->rope_caches && A->upload_rope == 0 && !g.prope[A->rope_slot].p) return DQ_ERR_INVALID_ARG;
    if (!stream()) return DQ_ERR_IO;
    const size_t E = A->n_embd, NT = A->n_total;
    const int slot = A->rope_caches ? A->rope_slot : 0;
    const LayerExtras ex =
        extras_of(A->bq, A->bk, A->bv, A->q_norm_w, A->k_norm_w, A->post_attn_norm_w, A->post_ffn_norm_w, A->q_dim,
                  A->kv_dim, A->head_dim, A->n_embd);
    if (!reserve(g.px, NT * E * 4) || !reserve(g.pwork, wbytes) ||
        !reserve(g.pnorm, 2 * dq_align256(E * 4) + ex.bytes()) ||
        (A->rope_caches && !reserve(g.prope[slot], NT * A->n_rot * 4)))
        return DQ_ERR_IO;
    const hipStream_t s = g.stream;
    if (A->upload_x) {
        g.mirror.clear();  // left over by a prompt that stopped midway
        if (hipMemcpyAsync(g.px.p, A->x, NT * E * 4, hipMemcpyHostToDevice, s) != hipSuccess) return io_fail();
    }
    if (A->rope_caches && A->upload_rope &&
        hipMemcpyAsync(g.prope[slot].p, A->rope_caches, NT * A->n_rot * 4, hipMemcpyHostToDevice, s) != hipSuccess)
        return io_fail();
    float* an = (float*)g.pnorm.p;
    float* fn = (float*)((uint8_t*)g.pnorm.p + dq_align256(E * 4));
    if (hipMemcpyAsync(an, A->attn_norm_w, E * 4, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipMemcpyAsync(fn, A->ffn_norm_w, E * 4, hipMemcpyHostToDevice, s) != hipSuccess ||
        !ex.upload(L, (uint8_t*)g.pnorm.p + 2 * dq_align256(E * 4), s))
        return io_fail();
    L.attn_norm = an;
    L.ffn_norm = fn;
    float* xc = (float*)g.px.p + (size_t)A->x_row0 * E;  // this chunk's rows, updated in place
    const float* rope = A->rope_caches ? (const float*)g.prope[slot].p + (size_t)A->x_row0 * A->n_rot : nullptr;
    const int rc = dq_layer_prefill(&L, xc, xc, rope, A->pos0, A->n_tok, A->n_swa, g.kc + A->kv_layer_off,
                                    g.vc + A->kv_layer_off, n_ctx, g.pwork.p, g.pwork.cap, s);
    if (rc != DQ_OK) return rc == DQ_ERR_IO ? io_fail() : rc;
    // the host cache follows the device rows (copied at the prompt's end)
    if (A->host_kcache && A->host_vcache) {
        const size_t off = A->kv_layer_off + (size_t)A->pos0 * pb;
        g.mirror.push_back({(uint8_t*)A->host_kcache + off, (uint8_t*)A->host_vcache + off, off, (size_t)A->n_tok * pb});
    }
    if (!A->download_x) return DQ_OK;
    for (const Engine::Mirror& m : g.mirror) {
        if (hipMemcpyAsync(m.k, g.kc + m.off, m.bytes, hipMemcpyDeviceToHost, s) != hipSuccess ||
            hipMemcpyAsync(m.v, g.vc + m.off, m.bytes, hipMemcpyDeviceToHost, s) != hipSuccess)
            return io_fail();
    }
    g.mirror.clear();
    const size_t r0 = A->x_out_row0 < A->n_total ? A->x_out_row0 : 0;
    if (hipMemcpyAsync(A->x_out + r0 * E, (float*)g.px.p + r0 * E, (NT - r0) * E * 4, hipMemcpyDeviceToHost, s) !=
        hipSuccess)
        return io_fail();
    return sync();
}

// Tokens per prefill chunk: 8 per CU (2048 on 256 CUs: the chunk's GEMMs
// fill the GPU with 128 x 256 tiles), within [1024, 4096].
int cuda_prefill_chunk_tokens(void) {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
        (void)hipGetLastError();
        return 0;
    }
    const int n = 8 * cus;
    return n < 1024 ? 1024 : (n > 4096 ? 4096 : n);
}

}  // extern "C"

// ------------------------------------------------------------------- head --

namespace {

bool sample_state_ready() {
    if (g.sst) return true;
    if (!stream()) return false;
    dq_sample_state_t* st = nullptr;
    if (hipMalloc((void**)&st, sizeof(dq_sample_state_t)) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    if (hipHostMalloc((void**)&g.tok_pinned, 4 * sizeof(int32_t), hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(st);
        g.tok_pinned = nullptr;
        return false;
    }
    bool ok = hipStreamCreateWithFlags(&g.tok_stream, hipStreamNonBlocking) == hipSuccess;
    for (int i = 0; ok && i < 4; ++i)
        ok = hipEventCreateWithFlags(&g.tok_ev[i], hipEventDisableTiming) == hipSuccess &&
             hipEventCreateWithFlags(&g.drawn_ev[i], hipEventDisableTiming) == hipSuccess;
    g.sst = st;
    if (!ok || dq_sample_reset(st, nullptr, 0, g.stream) != DQ_OK) {
        (void)hipGetLastError();
        return false;
    }
    return true;
}

// Final norm and head product of the token the layer chain left on the
// device, into g.hlog (backend_cuda.cu:3383-3436).
int head_launch(int format, const void* d_qs, const void* d_scale, const float* norm_w, size_t n_embd, float eps,
                size_t rows) {
    const WInfo* w = lookup(d_qs);
    if (!w || w->base != d_qs || w->fmt != format || w->rows != rows || w->cols != n_embd || !norm_w)
        return DQ_ERR_NOT_SUPPORTED;
    if (format == DQ_FMT_Q8_0 && (!d_scale || !lookup(d_scale) || lookup(d_scale)->base != d_qs))
        return DQ_ERR_NOT_SUPPORTED;
    if (!g.lx[g.cur].p || g.lx[g.cur].cap < n_embd * 4) return DQ_ERR_NOT_SUPPORTED;  // no device x
    if (n_embd % 4 || n_embd > 49152) return DQ_ERR_NOT_SUPPORTED;
    size_t wb = 0;
    if (dq_head_workspace_bytes(format, rows, n_embd, &wb) != DQ_OK) return DQ_ERR_NOT_SUPPORTED;
    if (!stream()) return DQ_ERR_IO;
    if (!reserve(g.hlog, rows * 4) || !reserve(g.hwork, wb) || !reserve(g.hnorm, n_embd * 4)) return DQ_ERR_IO;
    const hipStream_t s = g.stream;
    // the model's output norm, sent once; re-sent when its content changes
    // (a later model may reuse the host allocation)
    if (g.hnorm_host.size() != n_embd || memcmp(g.hnorm_host.data(), norm_w, n_embd * 4) != 0) {
        g.hnorm_host.assign(norm_w, norm_w + n_embd);
        if (hipMemcpyAsync(g.hnorm.p, g.hnorm_host.data(), n_embd * 4, hipMemcpyHostToDevice, s) != hipSuccess)
            return io_fail();
    }
    if (dq_head_logits(format, d_qs, rows, n_embd, (const float*)g.lx[g.cur].p, (const float*)g.hnorm.p, eps,
                       (float*)g.hlog.p, g.hwork.p, g.hwork.cap, s) != DQ_OK)
        return io_fail();
    return DQ_OK;
}

// The kk largest logits into g.hcand (ids then values).
int head_topk(size_t rows, uint32_t kk) {
    size_t tb = 0;
    if (rows > 0xFFFFFFFFu || dq_topk_workspace_bytes((uint32_t)rows, kk, &tb) != DQ_OK) return DQ_ERR_NOT_SUPPORTED;
    if (!reserve(g.htk, tb) || !reserve(g.hcand, 2 * 256 * 4)) return DQ_ERR_IO;
    int32_t* ids = (int32_t*)g.hcand.p;
    float* vals = (float*)g.hcand.p + 256;
    if (dq_topk((const float*)g.hlog.p, (uint32_t)rows, kk, ids, vals, g.htk.p, g.htk.cap, g.stream) != DQ_OK)
        return io_fail();
    return DQ_OK;
}

}  // namespace

extern "C" {

int cuda_head_forward(int format, const void* d_qs, const void* d_scale, const float* norm_w, size_t n_embd,
                      float eps, size_t rows, float* y) {
    if (!y) return DQ_ERR_INVALID_ARG;
    const int rc = head_launch(format, d_qs, d_scale, norm_w, n_embd, eps, rows);
    if (rc != DQ_OK) return rc;
    if (hipMemcpyAsync(y, g.hlog.p, rows * 4, hipMemcpyDeviceToHost, g.stream) != hipSuccess) return io_fail();
    return sync();
}

int cuda_head_forward_topk(int format, const void* d_qs, const void* d_scale, const float* norm_w, size_t n_embd,
                           float eps, size_t rows, uint32_t kk, int32_t* ids, float* vals) {
    if (kk == 0 || kk > 256 || rows < kk) return DQ_ERR_NOT_SUPPORTED;
    if (!ids || !vals) return DQ_ERR_INVALID_ARG;
    int rc = head_launch(format, d_qs, d_scale, norm_w, n_embd, eps, rows);
    if (rc == DQ_OK) rc = head_topk(rows, kk);
    if (rc != DQ_OK) return rc;
    const hipStream_t s = g.stream;
    if (hipMemcpyAsync(ids, g.hcand.p, kk * 4, hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipMemcpyAsync(vals, (float*)g.hcand.p + 256, kk * 4, hipMemcpyDeviceToHost, s) != hipSuccess)
        return io_fail();
    return sync();
}

int cuda_head_forward_sample(int format, const void* d_qs, const void* d_scale, const float* norm_w, size_t n_embd,
                             float eps, size_t rows, const CudaSampleArgs* a) {
    if (!a || a->kk == 0 || a->kk > 256 || rows < a->kk || a->slot > 3) return DQ_ERR_NOT_SUPPORTED;
    if (a->temperature > 0.0f && a->top_k <= 0) return DQ_ERR_NOT_SUPPORTED;
    if (a->penalty_last_n > DQ_SAMPLE_HIST) return DQ_ERR_NOT_SUPPORTED;
    if (!sample_state_ready()) return DQ_ERR_NOT_SUPPORTED;
    int rc = head_launch(format, d_qs, d_scale, norm_w, n_embd, eps, rows);
    if (rc == DQ_OK) rc = head_topk(rows, a->kk);
    if (rc != DQ_OK) return rc;
    const hipStream_t s = g.stream;
    if (dq_sample_candidates((const float*)g.hcand.p + 256, (const int32_t*)g.hcand.p, a->kk, a, g.sst, s) != DQ_OK)
        return io_fail();
    // the drawn token goes back on its own stream, so that the next step's
    // work on the decode stream does not wait for the copy
    const int slot = (int)a->slot;
    if (hipEventRecord(g.drawn_ev[slot], s) != hipSuccess ||
        hipStreamWaitEvent(g.tok_stream, g.drawn_ev[slot], 0) != hipSuccess ||
        hipMemcpyAsync(g.tok_pinned + slot, &g.sst->ring[slot], 4, hipMemcpyDeviceToHost, g.tok_stream) !=
            hipSuccess ||
        hipEventRecord(g.tok_ev[slot], g.tok_stream) != hipSuccess)
        return io_fail();
    return DQ_OK;
}

int cuda_sample_wait(uint32_t slot, int32_t* token) {
    if (slot > 3 || !token || !g.sst || !g.tok_ev[slot]) return DQ_ERR_IO;
    if (hipEventSynchronize(g.tok_ev[slot]) != hipSuccess) return io_fail();
    *token = g.tok_pinned[slot];
    return DQ_OK;
}

int cuda_sample_history(const int32_t* hist, size_t n) {
    if (!sample_state_ready()) return DQ_ERR_NOT_SUPPORTED;
    if (n && !hist) return DQ_ERR_INVALID_ARG;
    return dq_sample_reset(g.sst, hist, n, g.stream) == DQ_OK ? DQ_OK : io_fail();
}

int cuda_fetch_x(float* dst, size_t n) {
    if (!dst) return DQ_ERR_INVALID_ARG;
    if (!g.lx[g.cur].p || g.lx[g.cur].cap < n * 4 || !g.stream) return DQ_ERR_NOT_SUPPORTED;
    if (hipMemcpyAsync(dst, g.lx[g.cur].p, n * 4, hipMemcpyDeviceToHost, g.stream) != hipSuccess) return io_fail();
    return sync();
}

}  // extern "C"
