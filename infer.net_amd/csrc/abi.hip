// C ABI of libdeepinfer_hip (declared in include/deepinfer_hip.h). Every entry point
// validates all arguments before queuing GPU work (QuantizedTests.cs:118-135, 210-227).
#include <string.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <new>
#include <string>

#include "dih_internal.h"

// Fixed device scratch of dih_moe_decode_noalloc, the entry point for callers that cannot
// allocate. Every GPU holds its own copy at its own address for the life of the process.
// Host code never uses this name as a device pointer: the address of this device's copy
// comes from hipGetSymbolAddress (noalloc_scratch_address below) and is kept per device.
static constexpr size_t kNoAllocScratchBytes = 128 * 1024;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mutex;
bool g_noalloc_done[kMaxDevices];
void *g_noalloc_ptr[kMaxDevices];
hipError_t g_noalloc_rc[kMaxDevices];

// Device address of `scratch` on device `dev`, which must be the current device; looked up
// once per device.
void *noalloc_scratch_address(int dev, std::string &why) {
    if (dev < 0 || dev >= kMaxDevices) {
        why = "device index out of range for the no-allocation scratch";
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_noalloc_mutex);
    if (!g_noalloc_done[dev]) {
        void *ptr = nullptr;
        g_noalloc_rc[dev] = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        g_noalloc_ptr[dev] = g_noalloc_rc[dev] == hipSuccess ? ptr : nullptr;
        g_noalloc_done[dev] = true;
    }
    if (!g_noalloc_ptr[dev])
        why = std::string("no-allocation scratch lookup failed: ") + hipGetErrorString(g_noalloc_rc[dev]);
    return g_noalloc_ptr[dev];
}
}  // namespace

namespace dih {

void set_error(char *error, int capacity, const std::string &message) {
    if (error && capacity > 0) {
        size_t n = std::min(message.size(), (size_t)capacity - 1);
        memcpy(error, message.data(), n);
        error[n] = 0;
    }
}

bool hip_ok(hipError_t e, char *error, int capacity, const char *what) {
    if (e == hipSuccess) return true;
    set_error(error, capacity, std::string(what) + ": " + hipGetErrorString(e));
    return false;
}

void *ctx_scratch(Context *c, ScratchId id, size_t bytes, char *error, int capacity) {
    Scratch &s = c->ws[id];
    if (bytes == 0) bytes = 4;
    if (s.bytes >= bytes) return s.ptr;
    if (s.ptr) {
        // Growth is rare; make sure no queued kernel still uses the old block.
        if (!hip_ok(hipDeviceSynchronize(), error, capacity, "scratch sync")) return nullptr;
        (void)hipFree(s.ptr);
        s.ptr = nullptr;
        s.bytes = 0;
    }
    size_t rounded = (bytes + 255) & ~(size_t)255;
    if (!hip_ok(hipMalloc(&s.ptr, rounded), error, capacity, "scratch allocation")) return nullptr;
    if (!hip_ok(hipMemset(s.ptr, 0, rounded), error, capacity, "scratch clear")) return nullptr;
    s.bytes = rounded;
    return s.ptr;
}

bool sync_matrix(Matrix *m, char *error, int capacity) {
    for (int i = 0; i < 3; i++) {
        if (m->dirty[i] && m->host[i]) {
            if (!hip_ok(hipMemcpy(m->dev[i], m->host[i], m->bytes[i], hipMemcpyHostToDevice), error,
                        capacity, "weight upload"))
                return false;
            m->dirty[i] = false;
            if (i == 0 && !matrix_retile(m, 0, (size_t)m->experts * m->rows, error, capacity)) return false;
        }
    }
    // codes may have changed through the device pointer since it was handed out
    if (m->tiled_stale && !matrix_retile(m, 0, (size_t)m->experts * m->rows, error, capacity)) return false;
    return true;
}

static thread_local Context *tl_prof_ctx = nullptr;
static thread_local const char *tl_prof_name = "kernel";
static thread_local size_t tl_prof_first = 0;  // first record not yet named by prof_mark

ProfScope::ProfScope(Context *c) {
    tl_prof_ctx = c && c->profiling ? c : nullptr;
    tl_prof_name = "kernel";
    tl_prof_first = tl_prof_ctx ? tl_prof_ctx->prof_recs.size() : 0;
}
ProfScope::~ProfScope() { tl_prof_ctx = nullptr; }
void prof_stage(const char *name) { tl_prof_name = name; }

// Names the launches recorded since the previous mark (the kernels of one stage) that
// were not already named by prof_stage().
static void prof_mark(Context *c, hipStream_t, const char *name) {
    if (!c->profiling || tl_prof_ctx != c) return;
    for (size_t i = tl_prof_first; i < c->prof_recs.size(); i++)
        if (strcmp(c->prof_recs[i].name, "kernel") == 0) c->prof_recs[i].name = name;
    tl_prof_first = c->prof_recs.size();
}

static int prof_event(Context *c) {
    if (c->prof_used == (int)c->prof_pool.size()) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) return -1;
        c->prof_pool.push_back(e);
    }
    return c->prof_used++;
}

bool prof_events(hipEvent_t *start, hipEvent_t *stop) {
    Context *c = tl_prof_ctx;
    if (!c) return false;
    // Stream capture cannot hold these event pairs; launch normally while capturing.
    const int a = prof_event(c), b = prof_event(c);
    if (a < 0 || b < 0) return false;
    *start = c->prof_pool[a];
    *stop = c->prof_pool[b];
    c->prof_recs.push_back({a, b, tl_prof_name});
    return true;
}

static Context *as_ctx(void *p) {
    auto *c = static_cast<Context *>(p);
    return c && c->magic == 0x44494358u ? c : nullptr;
}
static Matrix *as_mat(void *p) {
    auto *m = static_cast<Matrix *>(p);
    return m && m->magic == 0x44494d58u ? m : nullptr;
}
// NULL selects the context's stream. That stream is a blocking one (hipStreamDefault), so
// its work is ordered after everything queued earlier on the null stream (torch's default
// stream) and before anything queued there later: a caller filling buffers on the null
// stream and then calling a dih_* entry point with stream NULL needs no synchronization.
static hipStream_t pick(Context *c, void *stream) {
    return stream ? static_cast<hipStream_t>(stream) : c->stream;
}

static bool stage(Matrix *m, size_t in_floats, size_t out_floats, char *error, int capacity) {
    if (m->stage_in_bytes < in_floats * 4) {
        if (m->stage_in) (void)hipFree(m->stage_in);
        m->stage_in = nullptr;
        m->stage_in_bytes = 0;
        if (!hip_ok(hipMalloc(&m->stage_in, in_floats * 4), error, capacity, "staging allocation")) return false;
        m->stage_in_bytes = in_floats * 4;
    }
    if (m->stage_out_bytes < out_floats * 4) {
        if (m->stage_out) (void)hipFree(m->stage_out);
        m->stage_out = nullptr;
        m->stage_out_bytes = 0;
        if (!hip_ok(hipMalloc(&m->stage_out, out_floats * 4), error, capacity, "staging allocation")) return false;
        m->stage_out_bytes = out_floats * 4;
    }
    return true;
}

static QmvSeg seg_of(const Matrix *m) {
    QmvSeg s;
    s.p0 = m->packed(); s.s0 = m->scales(); s.b0 = m->biases();
    s.rows = m->rows; s.columns = m->columns; s.experts = m->experts;
    return s;
}

static int cpl_of(int columns) { return (columns / 32 + 63) / 64; }

}  // namespace dih

using namespace dih;

extern "C" {

__attribute__((visibility("default"))) const char *dih_version(void) {
    return "deepinfer_hip 0.1 gfx950 (wave64, bf16 MFMA 32x32x16)";
}

__attribute__((visibility("default"))) void *dih_quant_create_configured(int resident, int refresh,
                                                                         char *error, int capacity) {
    if ((resident != 0 && resident != 1) || refresh < 0 || refresh > 60000) {
        set_error(error, capacity, "Invalid residency configuration");
        return nullptr;
    }
    int count = 0;
    if (!hip_ok(hipGetDeviceCount(&count), error, capacity, "device query")) return nullptr;
    if (count < 1) {
        set_error(error, capacity, "No HIP device");
        return nullptr;
    }
    int dev = 0;
    if (!hip_ok(hipGetDevice(&dev), error, capacity, "device query")) return nullptr;
    hipDeviceProp_t prop;
    if (!hip_ok(hipGetDeviceProperties(&prop, dev), error, capacity, "device query")) return nullptr;
    if (prop.warpSize != 64 || strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_error(error, capacity, std::string("Quantized kernels require gfx950 (wave64); found ") + prop.gcnArchName);
        return nullptr;
    }
    auto *c = new (std::nothrow) Context();
    if (!c) {
        set_error(error, capacity, "Out of host memory");
        return nullptr;
    }
    c->device = dev;
    c->resident = resident == 1;
    // a failed lookup only disables dih_moe_decode_noalloc (which then reports it)
    c->noalloc = noalloc_scratch_address(dev, c->noalloc_error);
    if (!hip_ok(hipStreamCreateWithFlags(&c->stream, hipStreamDefault), error, capacity, "stream") ||
        !hip_ok(hipEventCreate(&c->start), error, capacity, "event") ||
        !hip_ok(hipEventCreate(&c->stop), error, capacity, "event") ||
        !hip_ok(hipStreamCreateWithFlags(&c->side, hipStreamNonBlocking), error, capacity, "stream") ||
        !hip_ok(hipEventCreateWithFlags(&c->fork, hipEventDisableTiming), error, capacity, "event") ||
        !hip_ok(hipEventCreateWithFlags(&c->join, hipEventDisableTiming), error, capacity, "event")) {
        // release whatever was created before the failure
        for (hipEvent_t e : {c->start, c->stop, c->fork, c->join})
            if (e) (void)hipEventDestroy(e);
        for (hipStream_t st : {c->side, c->stream})
            if (st) (void)hipStreamDestroy(st);
        delete c;
        return nullptr;
    }
    return c;
}

__attribute__((visibility("default"))) void *dih_quant_create(char *error, int capacity) {
    return dih_quant_create_configured(0, 1000, error, capacity);
}

__attribute__((visibility("default"))) void dih_quant_destroy(void *p) {
    Context *c = as_ctx(p);
    if (!c) return;
    (void)hipStreamSynchronize(c->stream);
    for (auto &s : c->ws)
        if (s.ptr) (void)hipFree(s.ptr);
    for (auto &e : c->prof_pool) (void)hipEventDestroy(e);
    (void)hipEventDestroy(c->start);
    (void)hipEventDestroy(c->stop);
    (void)hipStreamSynchronize(c->side);
    (void)hipEventDestroy(c->fork);
    (void)hipEventDestroy(c->join);
    (void)hipStreamDestroy(c->side);
    (void)hipStreamDestroy(c->stream);
    c->magic = 0;
    delete c;
}

__attribute__((visibility("default"))) uint64_t dih_quant_residency_bytes(void *p) {
    Context *c = as_ctx(p);
    return c && c->resident ? c->weight_bytes : 0;
}

__attribute__((visibility("default"))) void dih_quant_residency_prepare(void *) {}

__attribute__((visibility("default"))) void *dih_quant_matrix_create(void *ctx, int experts, int rows,
                                                                     int columns, int bits, int group,
                                                                     char *error, int capacity) {
    Context *c = as_ctx(ctx);
    if (!c || experts < 1 || experts > 256 || rows < 1 || columns < 64 || columns > 8192 ||
        (bits != 5 && bits != 8) || group != 64 || columns % 64) {
        set_error(error, capacity, "Unsupported quantized matrix shape");
        return nullptr;
    }
    auto *m = new (std::nothrow) Matrix();
    if (!m) {
        set_error(error, capacity, "Out of host memory");
        return nullptr;
    }
    m->ctx = c;
    m->experts = experts; m->rows = rows; m->columns = columns; m->bits = bits;
    const size_t er = (size_t)experts * rows;
    m->bytes[0] = er * columns * bits / 8;
    m->bytes[1] = m->bytes[2] = er * (columns / 64) * 2;
    for (int i = 0; i < 3; i++) {
        if (hipMalloc(&m->dev[i], m->bytes[i]) != hipSuccess || hipMemset(m->dev[i], 0, m->bytes[i]) != hipSuccess) {
            for (int j = 0; j <= i; j++)
                if (m->dev[j]) (void)hipFree(m->dev[j]);
            delete m;
            set_error(error, capacity, "Quantized buffer allocation failed");
            return nullptr;
        }
    }
    // 5-bit matrices the streaming GEMM can take get the tile-major copy of their codes
    // (zeros, like the codes, until written)
    if (bits == 5 && columns % 512 == 0) {
        m->tiled_bytes = (size_t)experts * m->tiled_rows() * columns * bits / 8;
        if (hipMalloc(&m->tiled, m->tiled_bytes) != hipSuccess || hipMemset(m->tiled, 0, m->tiled_bytes) != hipSuccess) {
            if (m->tiled) (void)hipFree(m->tiled);
            for (int j = 0; j < 3; j++) (void)hipFree(m->dev[j]);
            delete m;
            set_error(error, capacity, "Quantized buffer allocation failed");
            return nullptr;
        }
    }
    c->weight_bytes += m->bytes[0] + m->bytes[1] + m->bytes[2] + m->tiled_bytes;
    return m;
}

__attribute__((visibility("default"))) void *dih_quant_matrix_buffer(void *matrix, int index) {
    Matrix *m = as_mat(matrix);
    if (!m || index < 0 || index > 2) return nullptr;
    if (!m->host[index]) {
        void *h = nullptr;
        if (hipHostMalloc(&h, m->bytes[index], hipHostMallocDefault) != hipSuccess) return nullptr;
        if (hipMemcpy(h, m->dev[index], m->bytes[index], hipMemcpyDeviceToHost) != hipSuccess) {
            (void)hipHostFree(h);
            return nullptr;
        }
        m->host[index] = h;
    }
    m->dirty[index] = true;
    return m->host[index];
}

__attribute__((visibility("default"))) void dih_quant_matrix_destroy(void *matrix) {
    Matrix *m = as_mat(matrix);
    if (!m) return;
    (void)hipDeviceSynchronize();
    if (m->ctx) m->ctx->weight_bytes -= m->bytes[0] + m->bytes[1] + m->bytes[2] + m->tiled_bytes;
    for (int i = 0; i < 3; i++) {
        if (m->dev[i]) (void)hipFree(m->dev[i]);
        if (m->host[i]) (void)hipHostFree(m->host[i]);
    }
    if (m->tiled) (void)hipFree(m->tiled);
    if (m->stage_in) (void)hipFree(m->stage_in);
    if (m->stage_out) (void)hipFree(m->stage_out);
    m->magic = 0;
    delete m;
}

__attribute__((visibility("default"))) int dih_quant_matrix_write(void *matrix, int index, size_t offset,
                                                                  const void *source, size_t bytes,
                                                                  char *error, int capacity) {
    Matrix *m = as_mat(matrix);
    if (!m || index < 0 || index > 2 || !source || offset > m->bytes[index] ||
        bytes > m->bytes[index] - offset) {
        set_error(error, capacity, "Invalid quantized buffer write");
        return -1;
    }
    if (!sync_matrix(m, error, capacity)) return -1;
    if (!hip_ok(hipMemcpy(static_cast<char *>(m->dev[index]) + offset, source, bytes, hipMemcpyDefault),
                error, capacity, "weight upload"))
        return -1;
    if (index == 0 && bytes > 0) {  // the code rows the write touched
        const size_t rb = m->words_per_row() * 4, r0 = offset / rb, r1 = (offset + bytes - 1) / rb + 1;
        if (!matrix_retile(m, r0, r1 - r0, error, capacity)) return -1;
    }
    if (m->host[index] && hipMemcpy(static_cast<char *>(m->host[index]) + offset, static_cast<char *>(m->dev[index]) + offset,
                                     bytes, hipMemcpyDeviceToHost) != hipSuccess) {
        set_error(error, capacity, "staging refresh failed");
        return -1;
    }
    return 0;
}

__attribute__((visibility("default"))) int dih_quant_matrix_commit(void *matrix, char *error, int capacity) {
    Matrix *m = as_mat(matrix);
    if (!m) {
        set_error(error, capacity, "Invalid matrix");
        return -1;
    }
    // codes written through the device pointer reach the tile-major copy here, and later
    // calls stop rewriting it
    if (!sync_matrix(m, error, capacity) || !matrix_retile(m, 0, (size_t)m->experts * m->rows, error, capacity))
        return -1;
    m->tiled_stale = false;
    for (int i = 0; i < 3; i++)
        if (m->host[i]) {
            (void)hipHostFree(m->host[i]);
            m->host[i] = nullptr;
        }
    return 0;
}

__attribute__((visibility("default"))) void *dih_quant_matrix_device(void *matrix, int index) {
    Matrix *m = as_mat(matrix);
    if (!m || index < 0 || index > 2) return nullptr;
    char err[8];
    if (!sync_matrix(m, err, sizeof(err))) return nullptr;
    // writes through the codes' pointer bypass the tile-major copy: keep it rewritten before
    // every use until the caller commits
    if (index == 0 && m->tiled) m->tiled_stale = true;
    return m->dev[index];
}

__attribute__((visibility("default"))) int dih_quant_matrix_shape(void *matrix, int *experts, int *rows,
                                                                  int *columns, int *bits) {
    Matrix *m = as_mat(matrix);
    if (!m) return -1;
    if (experts) *experts = m->experts;
    if (rows) *rows = m->rows;
    if (columns) *columns = m->columns;
    if (bits) *bits = m->bits;
    return 0;
}

// ---------------------------------------------------------------- host-pointer compute

__attribute__((visibility("default"))) int dih_quant_batch(void *ctx, const dih_job *jobs, int count,
                                                           double *ms, char *error, int capacity) {
    Context *c = as_ctx(ctx);
    if (!c || !jobs || count < 1 || count > 8) {
        set_error(error, capacity, "Invalid GEMV batch");
        return -1;
    }
    for (int j = 0; j < count; j++) {
        const dih_job &job = jobs[j];
        Matrix *m = as_mat(job.matrix);
        if (!m || m->ctx != c || !job.input || !job.output || !job.experts || job.count < 1 || job.count > 8) {
            set_error(error, capacity, "Invalid quantized GEMV arguments");
            return -1;
        }
        for (int i = 0; i < job.count; i++)
            if (job.experts[i] >= (uint32_t)m->experts) {
                set_error(error, capacity, "Expert ID out of bounds");
                return -1;
            }
        for (int i = 0; i < j; i++)
            if (jobs[i].matrix == job.matrix) {
                set_error(error, capacity, "Batch matrices must be distinct");
                return -1;
            }
    }
    uint32_t *ids = static_cast<uint32_t *>(ctx_scratch(c, S_IDS, 8 * 8 * 4, error, capacity));
    if (!ids) return -1;
    hipStream_t s = c->stream;
    for (int j = 0; j < count; j++) {
        Matrix *m = as_mat(jobs[j].matrix);
        size_t in_f = (size_t)m->columns * (jobs[j].batched ? jobs[j].count : 1);
        if (!sync_matrix(m, error, capacity) || !stage(m, in_f, (size_t)m->rows * jobs[j].count, error, capacity))
            return -1;
        if (!hip_ok(hipMemcpyAsync(m->stage_in, jobs[j].input, in_f * 4, hipMemcpyHostToDevice, s), error,
                    capacity, "input upload") ||
            !hip_ok(hipMemcpyAsync(ids + 8 * j, jobs[j].experts, jobs[j].count * 4, hipMemcpyHostToDevice, s),
                    error, capacity, "id upload"))
            return -1;
    }
    (void)hipEventRecord(c->start, s);
    // Jobs of equal bit width and chunk layout share one launch (up to four per launch).
    bool done[8] = {false};
    for (int j = 0; j < count; j++) {
        if (done[j]) continue;
        Matrix *mj = as_mat(jobs[j].matrix);
        QmvSeg segs[4];
        int n = 0;
        for (int k = j; k < count && n < 4; k++) {
            Matrix *mk = as_mat(jobs[k].matrix);
            if (done[k] || mk->bits != mj->bits || cpl_of(mk->columns) != cpl_of(mj->columns)) continue;
            QmvSeg sg = seg_of(mk);
            sg.ids = ids + 8 * k;
            sg.count = jobs[k].count;
            sg.x = mk->stage_in;
            sg.x_bf16 = 0;
            sg.x_slot_stride = jobs[k].batched ? mk->columns : 0;
            sg.y = mk->stage_out;
            segs[n++] = sg;
            done[k] = true;
        }
        if (!launch_qmv(segs, n, mj->bits, nullptr, s, error, capacity)) return -1;
    }
    (void)hipEventRecord(c->stop, s);
    if (!hip_ok(hipStreamSynchronize(s), error, capacity, "Quantized HIP command failed")) return -1;
    float elapsed = 0;
    (void)hipEventElapsedTime(&elapsed, c->start, c->stop);
    if (ms) *ms = elapsed;
    for (int j = 0; j < count; j++) {
        Matrix *m = as_mat(jobs[j].matrix);
        if (!hip_ok(hipMemcpy(jobs[j].output, m->stage_out, (size_t)m->rows * jobs[j].count * 4,
                              hipMemcpyDeviceToHost),
                    error, capacity, "output download"))
            return -1;
    }
    return 0;
}

__attribute__((visibility("default"))) int dih_quant_matvec(void *ctx, void *matrix, const float *x,
                                                            float *out, const uint32_t *experts, int count,
                                                            int batched, double *ms, char *error,
                                                            int capacity) {
    dih_job job{matrix, x, out, experts, count, batched};
    return dih_quant_batch(ctx, &job, 1, ms, error, capacity);
}

__attribute__((visibility("default"))) int dih_quant_experts(void *ctx, void *gate_, void *up_, void *down_,
                                                             void *shared_, const float *input,
                                                             const float *sharedInput,
                                                             const uint32_t *experts, int count,
                                                             float *expertOutput, float *sharedOutput,
                                                             double *ms, char *error, int capacity) {
    Context *c = as_ctx(ctx);
    Matrix *gate = as_mat(gate_), *up = as_mat(up_), *down = as_mat(down_), *shared = as_mat(shared_);
    if (!c || !gate || !up || !down || !shared || !input || !sharedInput || !experts || !expertOutput ||
        !sharedOutput || count < 1 || count > 8 || gate == up || gate == down || gate == shared ||
        up == down || up == shared || down == shared || gate->ctx != c || up->ctx != c ||
        down->ctx != c || shared->ctx != c || gate->rows != up->rows || gate->columns != up->columns ||
        gate->experts != up->experts || gate->bits != up->bits || down->experts != gate->experts ||
        down->columns != gate->rows || down->rows != gate->columns || shared->experts != 1 ||
        shared->rows != down->rows) {
        set_error(error, capacity, "Incompatible fused expert matrices/arguments");
        return -1;
    }
    for (int i = 0; i < count; i++)
        if (experts[i] >= (uint32_t)gate->experts) {
            set_error(error, capacity, "Expert ID out of bounds");
            return -1;
        }
    hipStream_t s = c->stream;
    const int I = gate->rows, H = down->rows;
    uint32_t *ids = static_cast<uint32_t *>(ctx_scratch(c, S_IDS, 8 * 8 * 4, error, capacity));
    float *act = static_cast<float *>(ctx_scratch(c, S_ACT, (size_t)8 * I * 4, error, capacity));
    if (!ids || !act) return -1;
    if (!sync_matrix(gate, error, capacity) || !sync_matrix(up, error, capacity) ||
        !sync_matrix(down, error, capacity) || !sync_matrix(shared, error, capacity) ||
        !stage(gate, gate->columns, 1, error, capacity) ||
        !stage(down, 1, (size_t)H * count, error, capacity) ||
        !stage(shared, shared->columns, H, error, capacity))
        return -1;
    if (!hip_ok(hipMemcpyAsync(gate->stage_in, input, (size_t)gate->columns * 4, hipMemcpyHostToDevice, s),
                error, capacity, "input upload") ||
        !hip_ok(hipMemcpyAsync(shared->stage_in, sharedInput, (size_t)shared->columns * 4,
                               hipMemcpyHostToDevice, s),
                error, capacity, "input upload") ||
        !hip_ok(hipMemcpyAsync(ids, experts, count * 4, hipMemcpyHostToDevice, s), error, capacity, "id upload"))
        return -1;
    (void)hipEventRecord(c->start, s);
    QmvSeg gu = seg_of(gate);
    gu.p1 = up->packed(); gu.s1 = up->scales(); gu.b1 = up->biases();
    gu.ids = ids; gu.count = count; gu.x = gate->stage_in; gu.y = act;
    if (!launch_qmv(&gu, 1, gate->bits, nullptr, s, error, capacity)) return -1;
    QmvSeg dn = seg_of(down);
    dn.ids = ids; dn.count = count; dn.x = act; dn.x_slot_stride = I; dn.y = down->stage_out;
    QmvSeg sh = seg_of(shared);
    sh.x = shared->stage_in; sh.y = shared->stage_out;
    if (down->bits == shared->bits && cpl_of(down->columns) == cpl_of(shared->columns)) {
        QmvSeg both[2] = {dn, sh};
        if (!launch_qmv(both, 2, down->bits, nullptr, s, error, capacity)) return -1;
    } else {
        if (!launch_qmv(&dn, 1, down->bits, nullptr, s, error, capacity) ||
            !launch_qmv(&sh, 1, shared->bits, nullptr, s, error, capacity))
            return -1;
    }
    (void)hipEventRecord(c->stop, s);
    if (!hip_ok(hipStreamSynchronize(s), error, capacity, "Quantized HIP command failed")) return -1;
    float elapsed = 0;
    (void)hipEventElapsedTime(&elapsed, c->start, c->stop);
    if (ms) *ms = elapsed;
    if (!hip_ok(hipMemcpy(expertOutput, down->stage_out, (size_t)H * count * 4, hipMemcpyDeviceToHost), error,
                capacity, "output download") ||
        !hip_ok(hipMemcpy(sharedOutput, shared->stage_out, (size_t)H * 4, hipMemcpyDeviceToHost), error,
                capacity, "output download"))
        return -1;
    return 0;
}

__attribute__((visibility("default"))) int dih_quant_embedding(void *matrix, int token, float *out) {
    Matrix *m = as_mat(matrix);
    if (!m || !out || token < 0 || token >= m->rows || m->experts != 1) return -1;
    char err[256];
    Context *c = m->ctx;
    float *dev = static_cast<float *>(ctx_scratch(c, S_STAGE_Y, (size_t)m->columns * 4, err, sizeof(err)));
    if (!dev || !sync_matrix(m, err, sizeof(err))) return -1;
    if (!launch_embedding(m, token, dev, c->stream, err, sizeof(err))) return -1;
    if (hipStreamSynchronize(c->stream) != hipSuccess) return -1;
    if (hipMemcpy(out, dev, (size_t)m->columns * 4, hipMemcpyDeviceToHost) != hipSuccess) return -1;
    return 0;
}

// ---------------------------------------------------------------- device-resident path

__attribute__((visibility("default"))) int dih_qmv(void *ctx, void *matrix, const void *x, int x_dtype, void *y,
                                                   int y_dtype, const uint32_t *experts, int count,
                                                   int batched, void *stream, char *error, int capacity) {
    Context *c = as_ctx(ctx);
    Matrix *m = as_mat(matrix);
    if (!c || !m || m->ctx != c || !x || !y || count < 1 || count > 8 || (x_dtype != DIH_F32 && x_dtype != DIH_BF16) ||
        (y_dtype != DIH_F32 && y_dtype != DIH_BF16) || (!experts && count != 1)) {
        set_error(error, capacity, "Invalid qmv arguments");
        return -1;
    }
    if (!sync_matrix(m, error, capacity)) return -1;
    QmvSeg sg = seg_of(m);
    sg.ids = experts; sg.count = count; sg.x = x; sg.x_bf16 = x_dtype == DIH_BF16;
    sg.x_slot_stride = batched ? m->columns : 0; sg.y = y; sg.y_bf16 = y_dtype == DIH_BF16;
    hipStream_t s = pick(c, stream);
    ProfScope prof_scope(c);
    bool ok = launch_qmv(&sg, 1, m->bits, nullptr, s, error, capacity);
    prof_mark(c, s, "qmv");
    return ok ? 0 : -1;
}

__attribute__((visibility("default"))) int dih_qmv_swiglu(void *ctx, void *gate_, void *up_, const void *x,
                                                          int x_dtype, float *act, const uint32_t *experts,
                                                          int count, void *stream, char *error, int capacity) {
    Context *c = as_ctx(ctx);
    Matrix *gate = as_mat(gate_), *up = as_mat(up_);
    if (!c || !gate || !up || gate == up || gate->ctx != c || up->ctx != c || gate->rows != up->rows ||
        gate->columns != up->columns || gate->experts != up->experts || gate->bits != up->bits || !x || !act ||
        count < 1 || count > 8 || (!experts && count != 1) || (x_dtype != DIH_F32 && x_dtype != DIH_BF16)) {
        set_error(error, capacity, "Invalid SwiGLU GEMV arguments");
        return -1;
    }
    if (!sync_matrix(gate, error, capacity) || !sync_matrix(up, error, capacity)) return -1;
    QmvSeg sg = seg_of(gate);
    sg.p1 = up->packed(); sg.s1 = up->scales(); sg.b1 = up->biases();
    sg.ids = experts; sg.count = count; sg.x = x; sg.x_bf16 = x_dtype == DIH_BF16; sg.y = act;
    hipStream_t s = pick(c, stream);
    ProfScope prof_scope(c);
    bool ok = launch_qmv(&sg, 1, gate->bits, nullptr, s, error, capacity);
    prof_mark(c, s, "qmv_swiglu");
    return ok ? 0 : -1;
}

__attribute__((visibility("default"))) int dih_argmax(void *ctx, const float *values, int n, uint32_t *next,
                                                      void *stream, char *error, int capacity) {
    Context *c = as_ctx(ctx);
    if (!c || !values || !next || n < 1) {
        set_error(error, capacity, "Invalid argmax arguments");
        return -1;
    }
    const size_t parts = (size_t)(n + kArgmaxPer - 1) / kArgmaxPer;
    float *pv = static_cast<float *>(ctx_scratch(c, S_ARGVAL, parts * 4, error, capacity));
    uint32_t *pi = static_cast<uint32_t *>(ctx_scratch(c, S_ARGIDX, parts * 4, error, capacity));
    if (!pv || !pi) return -1;
    hipStream_t s = pick(c, stream);
    return launch_argmax(values, n, pv, pi, next, s, error, capacity) ? 0 : -1;
}

__attribute__((visibility("default"))) int dih_lm_head(void *ctx, void *const *slices, int slice_count,
                                                       const void *x, float *logits, uint32_t *next,
                                                       void *stream, char *error, int capacity) {
    Context *c = as_ctx(ctx);
    if (!c || !slices || slice_count < 1 || slice_count > 64 || !x || !logits || !next) {
        set_error(error, capacity, "Invalid lm_head arguments");
        return -1;
    }
    Matrix *first = as_mat(slices[0]);
    long total = 0;
    for (int i = 0; i < slice_count; i++) {
        Matrix *m = as_mat(slices[i]);
        if (!m || !first || m->ctx != c || m->experts != 1 || m->columns != first->columns || m->bits != first->bits) {
            set_error(error, capacity, "lm_head slices must be single-expert matrices of equal width and bits");
            return -1;
        }
        total += m->rows;
    }
    if (total > 0x7fffffffL) {
        set_error(error, capacity, "Vocabulary too large");
        return -1;
    }
    for (int i = 0; i < slice_count; i++)
        if (!sync_matrix(as_mat(slices[i]), error, capacity)) return -1;
    const size_t parts = (size_t)(total + kArgmaxPer - 1) / kArgmaxPer;
    float *pv = static_cast<float *>(ctx_scratch(c, S_ARGVAL, parts * 4, error, capacity));
    uint32_t *pi = static_cast<uint32_t *>(ctx_scratch(c, S_ARGIDX, parts * 4, error, capacity));
    if (!pv || !pi) return -1;
    hipStream_t s = pick(c, stream);
    ProfScope prof_scope(c);
    long offset = 0;
    for (int i = 0; i < slice_count; i += 4) {
        QmvSeg segs[4];
        int n = 0;
        for (int k = i; k < slice_count && k < i + 4; k++) {
            Matrix *m = as_mat(slices[k]);
            QmvSeg sg = seg_of(m);
            sg.x = x; sg.x_bf16 = 1; sg.y = logits + offset;
            offset += m->rows;
            segs[n++] = sg;
        }
        if (!launch_qmv(segs, n, first->bits, nullptr, s, error, capacity)) return -1;
    }
    prof_mark(c, s, "lm_head_qmv");
    if (!launch_argmax(logits, (int)total, pv, pi, next, s, error, capacity)) return -1;
    prof_mark(c, s, "argmax");
    return 0;
}

__attribute__((visibility("default"))) int dih_top8(void *ctx, const void *logits, int logits_dtype, int tokens,
                                                    int experts, uint32_t *ids, float *probs, uint32_t *status,
                                                    void *stream, char *error, int capacity) {
    Context *c = as_ctx(ctx);
    if (!c || !logits || !ids || !probs || tokens < 1 || experts < 8 || experts > 256 ||
        (logits_dtype != DIH_F32 && logits_dtype != DIH_BF16)) {
        set_error(error, capacity, "Invalid router selection arguments");
        return -1;
    }
    return launch_top8(logits, logits_dtype == DIH_BF16, tokens, experts, ids, probs, status, nullptr,
                       nullptr, pick(c, stream), error, capacity)
               ? 0
               : -1;
}

__attribute__((visibility("default"))) int dih_build_groups(void *ctx, const uint32_t *ids, int tokens,
                                                            int experts, uint32_t *counts, uint32_t *routes,
                                                            void *stream, char *error, int capacity) {
    Context *c = as_ctx(ctx);
    if (!c || !ids || !counts || !routes || tokens < 1 || experts < 1 || experts > 256) {
        set_error(error, capacity, "Invalid grouping arguments");
        return -1;
    }
    return launch_build_groups(ids, tokens, experts, 0, counts, routes, pick(c, stream), error, capacity) ? 0 : -1;
}

__attribute__((visibility("default"))) int dih_dequant_bf16(void *ctx, void *matrix, int expert, uint16_t *out,
                                                            void *stream, char *error, int capacity) {
    Context *c = as_ctx(ctx);
    Matrix *m = as_mat(matrix);
    if (!c || !m || m->ctx != c || !out || expert < 0 || expert >= m->experts) {
        set_error(error, capacity, "Invalid dequantize arguments");
        return -1;
    }
    if (!sync_matrix(m, error, capacity)) return -1;
    return launch_dequant_bf16(m, expert, out, pick(c, stream), error, capacity) ? 0 : -1;
}

static bool check_layer(Context *c, const dih_moe_layer *L, bool need_router, int *E, int *H, int *I, int *Is,
                        char *error, int capacity) {
    if (!L) {
        set_error(error, capacity, "Missing MoE layer");
        return false;
    }
    Matrix *gate = as_mat(L->gate), *up = as_mat(L->up), *down = as_mat(L->down);
    Matrix *sg = as_mat(L->shared_gate), *su = as_mat(L->shared_up), *sd = as_mat(L->shared_down);
    Matrix *sr = as_mat(L->shared_route), *router = as_mat(L->router);
    if (!gate || !up || !down || !sg || !su || !sd || !sr || (need_router && !router) || (L->router && !router)) {
        set_error(error, capacity, "Incomplete MoE layer");
        return false;
    }
    Matrix *all[8] = {gate, up, down, sg, su, sd, sr, router};
    for (Matrix *m : all)
        if (m && m->ctx != c) {
            set_error(error, capacity, "MoE matrices must belong to this context");
            return false;
        }
    *E = gate->experts; *H = gate->columns; *I = gate->rows; *Is = sg->rows;
    if (up->experts != *E || up->rows != *I || up->columns != *H || up->bits != gate->bits ||
        down->experts != *E || down->rows != *H || down->columns != *I || down->bits != gate->bits ||
        sg->experts != 1 || su->experts != 1 || su->rows != *Is || sg->columns != *H || su->columns != *H ||
        su->bits != sg->bits || sd->experts != 1 || sd->rows != *H || sd->columns != *Is ||
        sr->experts != 1 || sr->rows != 1 || sr->columns != *H || *E < 8 ||
        (router && (router->experts != 1 || router->rows != *E || router->columns != *H)) || *I > 2048 ||
        *Is > 2048 || (*H % 64) != 0) {
        set_error(error, capacity, "Incompatible MoE layer shapes");
        return false;
    }
    for (Matrix *m : all)
        if (m && !sync_matrix(m, error, capacity)) return false;
    return true;
}

// dih_moe_merge -> MergeOut, validated (NULL = bf16 residual, no norm)
static bool merge_of(const dih_moe_merge *m, const void *residual, MergeOut &mo, char *error, int capacity) {
    mo = MergeOut();
    if (!m) return true;
    if ((m->residual_f32 != 0 && m->residual_f32 != 1) || (m->normed_f32 != 0 && m->normed_f32 != 1) ||
        (m->norm_weight && (!m->normed || m->normed == residual || !std::isfinite(m->epsilon) || m->epsilon <= 0.f))) {
        set_error(error, capacity, "Invalid MoE merge options");
        return false;
    }
    mo.residual_f32 = m->residual_f32;
    mo.norm_w = m->norm_weight;
    mo.eps = m->epsilon;
    mo.normed = m->normed;
    mo.normed_f32 = m->normed_f32;
    return true;
}

__attribute__((visibility("default"))) int dih_moe_decode(void *ctx, const dih_moe_layer *L, const void *x,
                                                          const float *logits, void *residual,
                                                          const dih_moe_trace *trace, void *stream, char *error,
                                                          int capacity) {
    return dih_moe_decode_norm(ctx, L, x, logits, residual, nullptr, trace, stream, error, capacity);
}

namespace dih {
// Device buffers of one decode MoE step (all fully written before they are read, so none
// needs clearing): logits [E], shared route [1], shared SwiGLU [Is], slot SwiGLU [8*I],
// shared down [H], ids [8], probs [8], status [1].
struct DecodeBuffers {
    float *lg, *srt, *sact, *act, *sout, *probs;
    uint32_t *ids, *status;
};

// Carves the step's buffers from `base` at 256-byte boundaries; returns the bytes used.
static size_t carve_decode(unsigned char *base, int E, int H, int I, int Is, DecodeBuffers &b) {
    size_t off = 0;
    auto take = [&](size_t bytes) {
        unsigned char *p = base ? base + off : nullptr;
        off += (bytes + 255) & ~(size_t)255;
        return p;
    };
    b.lg = reinterpret_cast<float *>(take((size_t)E * 4));
    b.srt = reinterpret_cast<float *>(take(16));
    b.sact = reinterpret_cast<float *>(take((size_t)Is * 4));
    b.act = reinterpret_cast<float *>(take((size_t)8 * I * 4));
    b.sout = reinterpret_cast<float *>(take((size_t)H * 4));
    b.ids = reinterpret_cast<uint32_t *>(take(8 * 8 * 4));
    b.probs = reinterpret_cast<float *>(take(8 * 4));
    b.status = reinterpret_cast<uint32_t *>(take(16));
    return off;
}

// The decode MoE step. `fixed` null: buffers from the context's grow-only scratch (which
// may allocate) and per-stage profiling; otherwise buffers carved from `fixed` (at most
// `fixed_bytes`) with no allocation and no profiling events.
static int moe_decode(Context *c, const dih_moe_layer *L, const void *x, const float *logits, void *residual,
                      const dih_moe_merge *merge, const dih_moe_trace *trace, void *stream,
                      unsigned char *fixed, size_t fixed_bytes, char *error, int capacity) {
    int E, H, I, Is;
    MergeOut mo;
    if (!x || !residual) {
        set_error(error, capacity, "Invalid decode MoE arguments");
        return -1;
    }
    if (!merge_of(merge, residual, mo, error, capacity)) return -1;
    if (!check_layer(c, L, logits == nullptr, &E, &H, &I, &Is, error, capacity)) return -1;
    if (logits && L->router) {
        set_error(error, capacity, "Pass either a router matrix or logits, not both");
        return -1;
    }
    Matrix *gate = as_mat(L->gate), *up = as_mat(L->up), *down = as_mat(L->down);
    Matrix *sg = as_mat(L->shared_gate), *su = as_mat(L->shared_up), *sd = as_mat(L->shared_down);
    Matrix *sr = as_mat(L->shared_route), *router = as_mat(L->router);
    DecodeBuffers bufs;
    if (fixed) {
        const size_t need = carve_decode(nullptr, E, H, I, Is, bufs);
        if (need > fixed_bytes) {
            set_error(error, capacity, "Decode MoE step needs " + std::to_string(need) +
                                           " bytes of scratch; the no-allocation scratch holds " +
                                           std::to_string(fixed_bytes));
            return -1;
        }
        carve_decode(fixed, E, H, I, Is, bufs);
    } else {
        bufs.lg = static_cast<float *>(ctx_scratch(c, S_LOGITS, (size_t)E * 4, error, capacity));
        bufs.srt = static_cast<float *>(ctx_scratch(c, S_SROUTE, 16, error, capacity));
        bufs.sact = static_cast<float *>(ctx_scratch(c, S_SACT, (size_t)Is * 4, error, capacity));
        bufs.act = static_cast<float *>(ctx_scratch(c, S_ACT, (size_t)8 * I * 4, error, capacity));
        bufs.sout = static_cast<float *>(ctx_scratch(c, S_SOUT, (size_t)H * 4, error, capacity));
        bufs.ids = static_cast<uint32_t *>(ctx_scratch(c, S_IDS, 8 * 8 * 4, error, capacity));
        bufs.probs = static_cast<float *>(ctx_scratch(c, S_PROBS, 8 * 4, error, capacity));
        bufs.status = static_cast<uint32_t *>(ctx_scratch(c, S_STATUS, 16, error, capacity));
        if (!bufs.lg || !bufs.srt || !bufs.sact || !bufs.act || !bufs.sout || !bufs.ids || !bufs.probs ||
            !bufs.status)
            return -1;
    }
    float *lg = bufs.lg, *srt = bufs.srt, *sact = bufs.sact, *act = bufs.act, *sout = bufs.sout;
    uint32_t *ids = bufs.ids;
    float *probs = bufs.probs;
    hipStream_t s = pick(c, stream);
    ProfScope prof_scope(fixed ? nullptr : c);
    if (decode_fast_path_ok(router, gate, down, sg, sd, sr)) {
        DecodeLaunch a;
        a.router = router; a.gate = gate; a.up = up; a.down = down;
        a.shared_gate = sg; a.shared_up = su; a.shared_down = sd; a.shared_route = sr;
        a.logits_in = logits;
        a.logits = trace && trace->logits ? trace->logits : lg;
        a.sact = sact; a.sroute = srt; a.act = act;
        a.ids = trace && trace->ids ? trace->ids : ids;
        a.probs = trace && trace->probs ? trace->probs : probs;
        a.status = trace ? trace->status : nullptr;
        a.x = static_cast<const uint16_t *>(x);
        a.residual = residual;
        a.residual_f32 = mo.residual_f32;
        a.route_out = trace ? trace->expert_out : nullptr;
        bool ok = launch_moe_decode(a, s, error, capacity);
        if (ok && mo.norm_w) {
            prof_stage("decode_norm");
            ok = launch_rmsnorm(residual, mo.residual_f32, 1, H, mo.norm_w, mo.eps, mo.normed, mo.normed_f32, a.probs, s,
                                error, capacity);
        }
        prof_stage("kernel");
        return ok ? 0 : -1;
    }
    const float *use_logits = logits ? logits : lg;
    // Stage 1: router logits, shared-expert gate GEMV and shared gate/up SwiGLU share x;
    // the last block of the launch that holds the router selects the experts.
    QmvSeg s1[3];
    int n8 = 0;
    Top8Source tp;
    tp.logits = use_logits; tp.experts = E; tp.ids = ids; tp.probs = probs; tp.status = trace ? trace->status : nullptr;
    if (router) {
        QmvSeg a = seg_of(router);
        a.x = x; a.x_bf16 = 1; a.y = lg;
        s1[n8++] = a;
    }
    QmvSeg b = seg_of(sr);
    b.x = x; b.x_bf16 = 1; b.y = srt;
    QmvSeg g = seg_of(sg);
    g.p1 = su->packed(); g.s1 = su->scales(); g.b1 = su->biases(); g.x = x; g.x_bf16 = 1; g.y = sact;
    // Group segments by bit width (router and shared_route are 8-bit; experts may be 5-bit).
    QmvSeg rest[2];
    int nrest = 0;
    if (sr->bits == 8) s1[n8++] = b; else rest[nrest++] = b;
    if (sg->bits == 8) s1[n8++] = g; else rest[nrest++] = g;
    if (n8 && !launch_qmv(s1, n8, 8, nullptr, s, error, capacity)) return -1;
    if (nrest && !launch_qmv(rest, nrest, 5, nullptr, s, error, capacity)) return -1;
    prof_mark(c, s, "decode_router_shared");
    // Stage 2: every wave selects the top-8 from the logits, then the selected experts'
    // gate/up SwiGLU; the shared down projection shares the launch.
    QmvSeg e2 = seg_of(gate);
    e2.p1 = up->packed(); e2.s1 = up->scales(); e2.b1 = up->biases();
    e2.top8 = 1; e2.count = 8; e2.x = x; e2.x_bf16 = 1; e2.y = act;
    QmvSeg d2 = seg_of(sd);
    d2.x = sact; d2.y = sout;
    if (sd->bits == gate->bits && cpl_of(sd->columns) == cpl_of(gate->columns)) {
        QmvSeg both[2] = {e2, d2};
        if (!launch_qmv(both, 2, gate->bits, &tp, s, error, capacity)) return -1;
    } else {
        if (!launch_qmv(&e2, 1, gate->bits, &tp, s, error, capacity) ||
            !launch_qmv(&d2, 1, sd->bits, nullptr, s, error, capacity))
            return -1;
    }
    prof_mark(c, s, "decode_experts_gate_up");
    // Stage 3: expert down projections and the weighted merge into the residual.
    if (!launch_moe_down_merge(down, act, ids, probs, sout, srt, residual, mo.residual_f32,
                               trace ? trace->expert_out : nullptr, s, error, capacity))
        return -1;
    prof_mark(c, s, "decode_down_merge");
    if (mo.norm_w) {
        if (!launch_rmsnorm(residual, mo.residual_f32, 1, H, mo.norm_w, mo.eps, mo.normed, mo.normed_f32, probs, s, error,
                            capacity))
            return -1;
        prof_mark(c, s, "decode_norm");
    }
    if (trace) {
        if (trace->logits && !hip_ok(hipMemcpyAsync(trace->logits, use_logits, (size_t)E * 4, hipMemcpyDeviceToDevice, s),
                                     error, capacity, "trace copy"))
            return -1;
        if (trace->ids && !hip_ok(hipMemcpyAsync(trace->ids, ids, 32, hipMemcpyDeviceToDevice, s), error, capacity,
                                  "trace copy"))
            return -1;
        if (trace->probs && !hip_ok(hipMemcpyAsync(trace->probs, probs, 32, hipMemcpyDeviceToDevice, s), error,
                                    capacity, "trace copy"))
            return -1;
    }
    return 0;
}
}  // namespace dih

__attribute__((visibility("default"))) int dih_moe_decode_norm(void *ctx, const dih_moe_layer *L, const void *x,
                                                               const float *logits, void *residual,
                                                               const dih_moe_merge *merge,
                                                               const dih_moe_trace *trace, void *stream,
                                                               char *error, int capacity) {
    Context *c = as_ctx(ctx);
    if (!c) {
        set_error(error, capacity, "Invalid decode MoE arguments");
        return -1;
    }
    return moe_decode(c, L, x, logits, residual, merge, trace, stream, nullptr, 0, error, capacity);
}

__attribute__((visibility("default"))) int dih_moe_decode_noalloc(void *ctx, const dih_moe_layer *L, const void *x,
                                                                  const float *logits, void *residual,
                                                                  const dih_moe_merge *merge,
                                                                  const dih_moe_trace *trace, void *stream,
                                                                  char *error, int capacity) {
    Context *c = as_ctx(ctx);
    if (!c) {
        set_error(error, capacity, "Invalid decode MoE arguments");
        return -1;
    }
    if (!c->noalloc) {
        set_error(error, capacity, c->noalloc_error);
        return -1;
    }
    return moe_decode(c, L, x, logits, residual, merge, trace, stream, static_cast<unsigned char *>(c->noalloc),
                      kNoAllocScratchBytes, error, capacity);
}

__attribute__((visibility("default"))) int dih_moe_prefill(void *ctx, const dih_moe_layer *L, int tokens,
                                                           const void *x, const void *logits, int logits_dtype,
                                                           void *residual, const dih_moe_trace *trace,
                                                           void *stream, char *error, int capacity) {
    return dih_moe_prefill_norm(ctx, L, tokens, x, logits, logits_dtype, residual, nullptr, trace, stream, error,
                                capacity);
}

__attribute__((visibility("default"))) int dih_moe_prefill_norm(void *ctx, const dih_moe_layer *L, int tokens,
                                                                const void *x, const void *logits,
                                                                int logits_dtype, void *residual,
                                                                const dih_moe_merge *merge,
                                                                const dih_moe_trace *trace, void *stream,
                                                                char *error, int capacity) {
    Context *c = as_ctx(ctx);
    int E, H, I, Is;
    MergeOut mo;
    if (!c || !x || !logits || !residual || tokens < 1 || tokens > (1 << 20) ||
        (logits_dtype != DIH_F32 && logits_dtype != DIH_BF16)) {
        set_error(error, capacity, "Invalid prefill MoE arguments");
        return -1;
    }
    if (!merge_of(merge, residual, mo, error, capacity)) return -1;
    if (!check_layer(c, L, false, &E, &H, &I, &Is, error, capacity)) return -1;
    Matrix *gate = as_mat(L->gate), *up = as_mat(L->up), *down = as_mat(L->down);
    Matrix *sg = as_mat(L->shared_gate), *su = as_mat(L->shared_up), *sd = as_mat(L->shared_down);
    Matrix *sr = as_mat(L->shared_route);
    if (Is != I || sg->bits != gate->bits || sd->bits != gate->bits) {
        set_error(error, capacity, "Grouped prefill needs the shared expert to match the routed experts' shape and bits");
        return -1;
    }
    const size_t T = (size_t)tokens, routes_n = T * 9;
    uint32_t *ids = static_cast<uint32_t *>(ctx_scratch(c, S_IDS, std::max<size_t>(T * 8 * 4, 256), error, capacity));
    float *probs = static_cast<float *>(ctx_scratch(c, S_PROBS, T * 8 * 4, error, capacity));
    uint32_t *counts = static_cast<uint32_t *>(ctx_scratch(c, S_COUNTS, (size_t)(E + 1) * 4, error, capacity));
    uint32_t *routes = static_cast<uint32_t *>(ctx_scratch(c, S_ROUTES, (size_t)(E + 1) * T * 4, error, capacity));
    uint16_t *actb = static_cast<uint16_t *>(ctx_scratch(c, S_ACTBF, routes_n * I * 2, error, capacity));
    float *rout = static_cast<float *>(ctx_scratch(c, S_ROUTEOUT, routes_n * H * 4, error, capacity));
    if (!ids || !probs || !counts || !routes || !actb || !rout) return -1;
    float *route_out = trace && trace->expert_out ? trace->expert_out : rout;
    hipStream_t s = pick(c, stream);
    ProfScope prof_scope(c);
    if (!launch_top8(logits, logits_dtype == DIH_BF16, tokens, E, ids, probs, trace ? trace->status : nullptr,
                     trace ? trace->logits : nullptr, nullptr, s, error, capacity))
        return -1;
    prof_mark(c, s, "prefill_top8");
    if (!launch_build_groups(ids, tokens, E, 1, counts, routes, s, error, capacity)) return -1;
    prof_mark(c, s, "prefill_group");
    // Wide 5-bit routing (the routed experts' gate/up work items fill whole rounds of the
    // GPU's one-block-a-CU slots): the shared expert's gate/up and down run as launches of
    // their own on a side stream, so that its items and the routed down projection fill the
    // tail of the routed gate/up instead of adding a round (config 4: 353-360 -> 339-341 us
    // over two graph-replayed steps, 371-372 -> 355-358 us over ten; 8-bit Zipf routing
    // measured slower so and keeps one launch for both)
    const bool beside = qmm_wide_gated(gate, tokens);
    hipStream_t ss = beside ? c->side : s;
    if (beside && (!hip_ok(hipEventRecord(c->fork, s), error, capacity, "event") ||
                   !hip_ok(hipStreamWaitEvent(ss, c->fork, 0), error, capacity, "event")))
        return -1;
    // (group E of routes/counts is the shared expert: route T*8 + t for token t)
    QmmArgs a;
    a.m0 = gate; a.m1 = up; a.tokens = tokens; a.routes = routes; a.counts = counts;
    a.ngroups = E + 1; a.x = static_cast<const uint16_t *>(x); a.in_mode = 1;
    a.y = actb; a.y_bf16 = 1;
    if (beside) a.ngroups = E;
    else { a.sm0 = sg; a.sm1 = su; }
    QmmArgs as = a;
    as.m0 = sg; as.m1 = su; as.sm0 = as.sm1 = nullptr;
    as.routes = routes + (size_t)E * T; as.counts = counts + E; as.ngroups = 1;
    QmmArgs d;
    d.m0 = down; d.tokens = tokens; d.routes = routes; d.counts = counts; d.ngroups = E + 1;
    d.x = actb; d.in_mode = 0; d.y = route_out; d.y_bf16 = 0;
    if (beside) d.ngroups = E;
    else d.sm0 = sd;
    QmmArgs ds = d;
    ds.m0 = sd; ds.sm0 = nullptr;
    ds.routes = routes + (size_t)E * T; ds.counts = counts + E; ds.ngroups = 1;
    bool ok = launch_qmm(a, s, error, capacity) && (!beside || launch_qmm(as, ss, error, capacity));
    if (ok) prof_mark(c, s, "prefill_gate_up");
    ok = ok && launch_qmm(d, s, error, capacity) && (!beside || launch_qmm(ds, ss, error, capacity));
    // the side stream joins back even after a failed launch, so that a stream under capture
    // is left with one branch
    if (beside) {
        char jerr[256];
        const bool joined = hip_ok(hipEventRecord(c->join, ss), jerr, sizeof(jerr), "event") &&
                            hip_ok(hipStreamWaitEvent(s, c->join, 0), jerr, sizeof(jerr), "event");
        if (ok && !joined) {
            set_error(error, capacity, jerr);
            ok = false;
        }
    }
    if (!ok) return -1;
    prof_mark(c, s, "prefill_down");
    if (!launch_moe_merge(sr, static_cast<const uint16_t *>(x), tokens, H, route_out, probs, residual, mo, s,
                          error, capacity))
        return -1;
    prof_mark(c, s, "prefill_merge");
    if (trace) {
        if (trace->ids && !hip_ok(hipMemcpyAsync(trace->ids, ids, T * 32, hipMemcpyDeviceToDevice, s), error,
                                  capacity, "trace copy"))
            return -1;
        if (trace->probs && !hip_ok(hipMemcpyAsync(trace->probs, probs, T * 32, hipMemcpyDeviceToDevice, s), error,
                                    capacity, "trace copy"))
            return -1;
    }
    return 0;
}

__attribute__((visibility("default"))) int dih_grouped_qmm(void *ctx, void *matrix, void *up_matrix, int tokens,
                                                           const void *x, int input_mode, const uint32_t *counts,
                                                           const uint32_t *routes, void *y, int y_dtype,
                                                           void *stream, char *error, int capacity) {
    Context *c = as_ctx(ctx);
    Matrix *m = as_mat(matrix), *up = up_matrix ? as_mat(up_matrix) : nullptr;
    if (!c || !m || m->ctx != c || (up_matrix && (!up || up->ctx != c || up == m)) || tokens < 1 ||
        tokens > (1 << 20) || !x || !counts || !routes || !y || (input_mode != 0 && input_mode != 1) ||
        (y_dtype != DIH_F32 && y_dtype != DIH_BF16)) {
        set_error(error, capacity, "Invalid grouped qmm arguments");
        return -1;
    }
    if (up && (up->experts != m->experts || up->rows != m->rows || up->columns != m->columns || up->bits != m->bits)) {
        set_error(error, capacity, "Gate and up matrices must share shape and bits");
        return -1;
    }
    if (!sync_matrix(m, error, capacity) || (up && !sync_matrix(up, error, capacity))) return -1;
    hipStream_t s = pick(c, stream);
    ProfScope prof_scope(c);
    QmmArgs a;
    a.m0 = m; a.m1 = up; a.tokens = tokens; a.routes = routes; a.counts = counts; a.ngroups = m->experts;
    a.x = static_cast<const uint16_t *>(x); a.in_mode = input_mode; a.y = y; a.y_bf16 = y_dtype == DIH_BF16;
    const bool ok = launch_qmm(a, s, error, capacity);
    prof_mark(c, s, up ? "grouped_gate_up" : "grouped_qmm");
    return ok ? 0 : -1;
}

__attribute__((visibility("default"))) int dih_dense(void *ctx, void *matrix, int tokens, const void *x, void *y,
                                                     int y_dtype, void *stream, char *error, int capacity) {
    Context *c = as_ctx(ctx);
    Matrix *m = as_mat(matrix);
    if (!c || !m || m->ctx != c || m->experts != 1 || tokens < 1 || !x || !y ||
        (y_dtype != DIH_F32 && y_dtype != DIH_BF16)) {
        set_error(error, capacity, "Invalid dense projection arguments");
        return -1;
    }
    if (!sync_matrix(m, error, capacity)) return -1;
    hipStream_t s = pick(c, stream);
    ProfScope prof_scope(c);
    // Dispatch policy (p_gemv, gpu_prefill.mm:603-620, picks GEMV kernels below 64 tokens):
    // up to kDenseGemvTokens tokens run as one batched GEMV launch (each token a slot of
    // expert 0; measured 8 / 13 / 18 us against 26 us for the MFMA tile at 1 / 2 / 4 tokens
    // of an 8192 x 2048 8-bit matrix), long chunks as the bf16 GEMM after one dequantization
    // pass (the fused tile re-dequantizes the weights for every 128 tokens), the rest as the
    // fused MFMA GEMM.
    constexpr int kDenseGemvTokens = 4;
    if (tokens >= 1024 || (tokens >= 512 && m->rows <= 4096)) {
        bool ok = launch_dense_gemm(c, m, tokens, static_cast<const uint16_t *>(x), y, y_dtype == DIH_BF16, s,
                                    error, capacity);
        prof_mark(c, s, "dense_qmm");
        return ok ? 0 : -1;
    }
    if (tokens <= kDenseGemvTokens) {
        QmvSeg sg = seg_of(m);
        sg.count = tokens; sg.x = x; sg.x_bf16 = 1; sg.x_slot_stride = m->columns;
        sg.y = y; sg.y_bf16 = y_dtype == DIH_BF16;
        bool ok = launch_qmv(&sg, 1, m->bits, nullptr, s, error, capacity);
        prof_mark(c, s, "dense_qmm");
        return ok ? 0 : -1;
    }
    QmmArgs a;
    a.m0 = m; a.tokens = tokens; a.dense = 1; a.x = static_cast<const uint16_t *>(x); a.in_mode = 0;
    a.y = y; a.y_bf16 = y_dtype == DIH_BF16;
    bool ok = launch_qmm(a, s, error, capacity);
    prof_mark(c, s, "dense_qmm");
    return ok ? 0 : -1;
}

__attribute__((visibility("default"))) int dih_attention(void *ctx, const void *q, int q_dtype,
                                                         const uint16_t *keys, const uint16_t *values,
                                                         int cache_positions, const void *gate, int gate_dtype,
                                                         void *out, int out_dtype, int position, int tokens,
                                                         int partition, void *stream, char *error, int capacity) {
    Context *c = as_ctx(ctx);
    auto dtype_ok = [](int d) { return d == DIH_F32 || d == DIH_BF16; };
    if (!c || !q || !keys || !values || !gate || !out || !dtype_ok(q_dtype) || !dtype_ok(gate_dtype) ||
        !dtype_ok(out_dtype) || tokens < 1 || position < 0 || cache_positions < 1 ||
        (int64_t)position + tokens > cache_positions || partition < 0 || partition % 32 != 0) {
        set_error(error, capacity, "Invalid attention arguments");
        return -1;
    }
    const int round = attention_partition(position, tokens, partition);
    const int part = attention_split(position, tokens, round);
    const size_t nparts = (size_t)attention_partials(position, tokens, part);
    AttentionArgs a;
    a.q = q; a.q_bf16 = q_dtype == DIH_BF16;
    a.keys = keys; a.values = values;
    a.gate = gate; a.gate_bf16 = gate_dtype == DIH_BF16;
    a.out = out; a.out_bf16 = out_dtype == DIH_BF16;
    a.position = position; a.tokens = tokens; a.partition = part; a.round = round;
    if (nparts > 1) {
        const size_t rows = (size_t)tokens * 16 * nparts;
        a.pacc = static_cast<float *>(ctx_scratch(c, S_APART, rows * 256 * 4, error, capacity));
        a.pstat = static_cast<float *>(ctx_scratch(c, S_ASTAT, rows * 8, error, capacity));
        if (!a.pacc || !a.pstat) return -1;
    }
    if (const size_t sf = attention_score_floats(position, tokens, round, part)) {
        a.scores = static_cast<float *>(ctx_scratch(c, S_ASCORE, sf * 4, error, capacity));
        if (!a.scores) return -1;
    }
    hipStream_t s = pick(c, stream);
    ProfScope prof_scope(c);
    bool ok = launch_attention(a, s, error, capacity);
    prof_mark(c, s, "attention");
    return ok ? 0 : -1;
}

__attribute__((visibility("default"))) int dih_delta_rule(void *ctx, float *state, float *history, const float *conv,
                                                          const float *decay, const float *beta, const float *raw,
                                                          float *out, int tokens, int path, void *stream,
                                                          char *error, int capacity) {
    Context *c = as_ctx(ctx);
    if (!c || !state || !history || !conv || !decay || !beta || !raw || !out || tokens < 1 ||
        tokens > (1 << 20) || path < 0 || path > 2) {
        set_error(error, capacity, "Invalid delta rule arguments");
        return -1;
    }
    DeltaArgs a;
    a.conv = conv; a.decay = decay; a.beta = beta; a.raw = raw;
    a.state = state; a.history = history; a.out = out; a.tokens = tokens;
    // p_delta (gpu_prefill.mm:540-551) switches to the chunkwise form at 64 tokens, which is
    // also where the two measured equal on MI355X (sequential 19.8 us vs chunkwise 20.1 us at
    // 56 tokens, 22.1 vs 20.0 us at 64)
    constexpr int kChunkwiseFrom = 64;
    a.chunked = path == 0 ? tokens >= kChunkwiseFrom : path == 2;
    if (a.chunked) {
        const size_t blocks = ((size_t)tokens + 31) / 32, tiles = blocks * 32;
        a.w = static_cast<float *>(ctx_scratch(c, S_DW, tiles * 32 * 128 * 4, error, capacity));
        a.u = static_cast<float *>(ctx_scratch(c, S_DU, tiles * 32 * 128 * 4, error, capacity));
        a.qp = static_cast<float *>(ctx_scratch(c, S_DQ, tiles * 32 * 128 * 4, error, capacity));
        a.cu = static_cast<float *>(ctx_scratch(c, S_DCU, tiles * 32 * 128 * 4, error, capacity));
        a.factors = static_cast<float *>(ctx_scratch(c, S_DF, tiles * 32 * 2 * 4, error, capacity));
        if (!a.w || !a.u || !a.qp || !a.cu || !a.factors) return -1;
    }
    hipStream_t s = pick(c, stream);
    ProfScope prof_scope(c);
    bool ok = launch_delta_rule(a, s, error, capacity);
    prof_mark(c, s, "delta");
    return ok ? 0 : -1;
}

// ---------------------------------------------------------------- host-pointer delta step

namespace dih {
// Device memory of one DeltaMemory (DeltaState, quantized.mm:21-23): the recurrent state
// and the staging of one token's operands, in one allocation.
struct DeltaState {
    Context *ctx = nullptr;
    float *block = nullptr;
    uint32_t magic = 0x44494453u;
    static constexpr size_t kState = 32 * 128 * 128, kConv = 8192, kHeads = 32, kOut = 4096;
    static constexpr size_t kHistory = 3 * 8192;
    static constexpr size_t kFloats = kState + kConv + 2 * kHeads + kOut + kHistory;
    float *state() const { return block; }
    float *conv() const { return block + kState; }          // q [2048], k [2048], v [4096]
    float *decay() const { return conv() + kConv; }
    float *beta() const { return decay() + kHeads; }
    float *out() const { return beta() + kHeads; }
    float *history() const { return out() + kOut; }         // unused roll target of the kernel
};
static DeltaState *as_delta(void *p) {
    auto *d = static_cast<DeltaState *>(p);
    return d && d->magic == 0x44494453u ? d : nullptr;
}
}  // namespace dih

__attribute__((visibility("default"))) void *dih_delta_create(void *ctx) {
    Context *c = as_ctx(ctx);
    if (!c) return nullptr;
    auto *d = new (std::nothrow) DeltaState();
    if (!d) return nullptr;
    d->ctx = c;
    if (hipMalloc(&d->block, DeltaState::kFloats * 4) != hipSuccess) {
        delete d;
        return nullptr;
    }
    // the state starts at zero (di_delta_create memsets it); the rest is zeroed as well so
    // that the kernel's history roll never reads uninitialized memory
    if (hipMemset(d->block, 0, DeltaState::kFloats * 4) != hipSuccess) {
        (void)hipFree(d->block);
        delete d;
        return nullptr;
    }
    return d;
}

__attribute__((visibility("default"))) void dih_delta_destroy(void *state) {
    DeltaState *d = as_delta(state);
    if (!d) return;
    (void)hipStreamSynchronize(d->ctx->stream);
    (void)hipFree(d->block);
    d->magic = 0;
    delete d;
}

__attribute__((visibility("default"))) int dih_delta_step(void *ctx, void *state, const float *q, const float *k,
                                                          const float *v, const float *decay, const float *beta,
                                                          float *out, double *ms, char *error, int capacity) {
    Context *c = as_ctx(ctx);
    DeltaState *d = as_delta(state);
    if (!c || !d || !q || !k || !v || !decay || !beta || !out) {
        set_error(error, capacity, "Null delta argument");
        return -1;
    }
    if (d->ctx != c) {
        set_error(error, capacity, "Delta state belongs to another context");
        return -1;
    }
    hipStream_t s = c->stream;
    if (!hip_ok(hipMemcpyAsync(d->conv(), q, 2048 * 4, hipMemcpyHostToDevice, s), error, capacity, "delta upload") ||
        !hip_ok(hipMemcpyAsync(d->conv() + 2048, k, 2048 * 4, hipMemcpyHostToDevice, s), error, capacity,
                "delta upload") ||
        !hip_ok(hipMemcpyAsync(d->conv() + 4096, v, 4096 * 4, hipMemcpyHostToDevice, s), error, capacity,
                "delta upload") ||
        !hip_ok(hipMemcpyAsync(d->decay(), decay, 32 * 4, hipMemcpyHostToDevice, s), error, capacity,
                "delta upload") ||
        !hip_ok(hipMemcpyAsync(d->beta(), beta, 32 * 4, hipMemcpyHostToDevice, s), error, capacity, "delta upload"))
        return -1;
    // one token of the sequential delta rule (delta_step, quantized.mm:191-212, is the same
    // recurrence); the raw rows of the history roll are the operands themselves
    DeltaArgs a;
    a.conv = d->conv(); a.decay = d->decay(); a.beta = d->beta(); a.raw = d->conv();
    a.state = d->state(); a.history = d->history(); a.out = d->out(); a.tokens = 1; a.chunked = 0;
    (void)hipEventRecord(c->start, s);
    if (!launch_delta_rule(a, s, error, capacity)) return -1;
    (void)hipEventRecord(c->stop, s);
    if (!hip_ok(hipStreamSynchronize(s), error, capacity, "Gated delta HIP command failed")) return -1;
    float elapsed = 0;
    (void)hipEventElapsedTime(&elapsed, c->start, c->stop);
    if (ms) *ms = elapsed;
    return hip_ok(hipMemcpy(out, d->out(), 4096 * 4, hipMemcpyDeviceToHost), error, capacity, "delta download")
               ? 0
               : -1;
}

__attribute__((visibility("default"))) int dih_attention_partition(int position, int tokens, int partition) {
    if (tokens < 1 || position < 0 || partition < 0 || partition % 32 != 0) return -1;
    return attention_partition(position, tokens, partition);
}

__attribute__((visibility("default"))) int dih_set_profiling(void *ctx, int enabled) {
    Context *c = as_ctx(ctx);
    if (!c) return -1;
    if (c->prof_used && hipDeviceSynchronize() != hipSuccess) return -1;
    c->profiling = enabled != 0;
    c->prof_recs.clear();
    c->prof_used = 0;
    return 0;
}

__attribute__((visibility("default"))) int dih_profile_read(void *ctx, double *total_ms, int *counts,
                                                            const char **names, int capacity) {
    Context *c = as_ctx(ctx);
    if (!c || !c->profiling) return 0;
    if (c->prof_used && hipEventSynchronize(c->prof_pool[c->prof_used - 1]) != hipSuccess) return -1;
    int n = 0;
    for (const auto &r : c->prof_recs) {
        int k = 0;
        while (k < n && strcmp(names[k], r.name) != 0) k++;
        if (k == n) {
            if (n == capacity) continue;
            names[n] = r.name;
            total_ms[n] = 0;
            counts[n] = 0;
            n++;
        }
        float e = 0;
        (void)hipEventElapsedTime(&e, c->prof_pool[r.begin], c->prof_pool[r.end]);
        total_ms[k] += e;
        counts[k] += 1;
    }
    return n;
}

}  // extern "C"
