// Checkpoint loading into device matrices: the safetensors reader (SafeTensors.cs:7-95) and
// the MLX-affine checkpoint layout of Qwen3.6-35B-A3B (Qwen36Weights.cs:26-122), with
// tensor bytes streamed file -> pinned staging -> HBM.
//
// Safetensors rules kept from the reference, in order: u64 little-endian header length in
// [2, 16 MiB] and within the file; a JSON object whose entries (except "__metadata__") have
// dtype BF16 / F32 / U32 (anything else is unsupported), rank 1..8 with every dim >= 1,
// data_offsets [begin, end] inside the data section with end - begin = elements * dtype
// size and elements <= INT32_MAX; no duplicate names; no overlapping byte ranges.
// Failures report -1 (invalid data, the reference's InvalidDataException) or -2
// (unsupported, NotSupportedException) plus the reference's message text.
//
// Upload: each tensor is read with pread (up to eight threads per 64 MiB piece) into one of
// two pinned 64 MiB staging buffers while the other is copied to the device on the
// checkpoint's own stream, so disk or page cache reads overlap the PCIe copies. No host-side staging copy of the whole matrix is
// kept (the reference writes into unified memory in place, QuantizedMetal.cs:177).
#include <fcntl.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <memory>
#include <thread>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "dih_internal.h"
#include "json.h"

namespace dih {

namespace {

enum { kOk = 0, kInvalid = -1, kUnsupported = -2 };
enum { kBF16 = 1, kF32 = 2, kU32 = 3 };

struct StTensor {
    std::string name;
    int dtype = 0;
    std::vector<int64_t> shape;
    int64_t start = 0, bytes = 0;
};

struct StFile {
    uint32_t magic = 0x44495354u;
    int fd = -1;
    int64_t size = 0, data_start = 0;
    std::vector<StTensor> tensors;  // header order
    std::unordered_map<std::string, size_t> by_name;
    ~StFile() {
        if (fd >= 0) ::close(fd);
        magic = 0;
    }
};

struct Failure {
    int code = kOk;
    std::string message;
    bool set(int c, const std::string &m) {
        code = c;
        message = m;
        return false;
    }
};

bool read_all(int fd, void *dst, size_t bytes, int64_t offset) {
    char *p = static_cast<char *>(dst);
    while (bytes) {
        const ssize_t n = ::pread(fd, p, bytes, (off_t)offset);
        if (n <= 0) return false;
        p += n;
        bytes -= (size_t)n;
        offset += n;
    }
    return true;
}

// Large reads in up to eight parallel pread streams (page-cache copies are bounded by one
// thread's memcpy rate; NVMe reads by queue depth).
bool read_parallel(int fd, void *dst, size_t bytes, int64_t offset) {
    constexpr size_t kPart = (size_t)8 << 20;
    const int parts = (int)std::min<size_t>(8, (bytes + kPart - 1) / kPart);
    if (parts <= 1) return read_all(fd, dst, bytes, offset);
    const size_t per = ((bytes + parts - 1) / parts + 4095) & ~(size_t)4095;
    std::atomic<bool> ok{true};
    std::vector<std::thread> th;
    for (int i = 1; i < parts; i++) {
        const size_t b = per * (size_t)i;
        if (b >= bytes) break;
        const size_t n = std::min(per, bytes - b);
        th.emplace_back([&, b, n] {
            if (!read_all(fd, static_cast<char *>(dst) + b, n, offset + (int64_t)b)) ok = false;
        });
    }
    if (!read_all(fd, dst, std::min(per, bytes), offset)) ok = false;
    for (auto &x : th) x.join();
    return ok;
}

int dtype_code(const std::string &d) {
    if (d == "BF16") return kBF16;
    if (d == "F32") return kF32;
    if (d == "U32") return kU32;
    return 0;
}
int dtype_bytes(int code) { return code == kBF16 ? 2 : 4; }

// SafeTensors.cs:13-44
StFile *st_open(const char *path, Failure &f) {
    std::unique_ptr<StFile> s(new (std::nothrow) StFile());
    if (!s) { f.set(kInvalid, "Out of host memory."); return nullptr; }
    s->fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (s->fd < 0) { f.set(kInvalid, std::string("Cannot open safetensors file: ") + path); return nullptr; }
    struct stat st;
    if (fstat(s->fd, &st) != 0) { f.set(kInvalid, "Cannot stat safetensors file."); return nullptr; }
    s->size = (int64_t)st.st_size;
    unsigned char lb[8];
    if (s->size < 8 || !read_all(s->fd, lb, 8, 0)) { f.set(kInvalid, "Invalid safetensors header length."); return nullptr; }
    uint64_t hl = 0;
    for (int i = 7; i >= 0; i--) hl = (hl << 8) | lb[i];
    if (hl < 2 || hl > 16777216 || hl > (uint64_t)(s->size - 8)) {
        f.set(kInvalid, "Invalid safetensors header length.");
        return nullptr;
    }
    std::string header((size_t)hl, '\0');
    if (!read_all(s->fd, &header[0], (size_t)hl, 8)) { f.set(kInvalid, "Invalid safetensors header length."); return nullptr; }
    s->data_start = 8 + (int64_t)hl;
    json::Value root;
    std::string err;
    if (!json::parse(header.data(), header.size(), root, err)) { f.set(kInvalid, err + "."); return nullptr; }
    if (root.type != json::Value::Object) { f.set(kInvalid, "Safetensors header is not an object."); return nullptr; }
    const int64_t data_bytes = s->size - s->data_start;
    for (const auto &entry : root.members) {
        if (entry.first == "__metadata__") continue;
        const json::Value &v = entry.second;
        const json::Value *dt = v.find("dtype"), *sh = v.find("shape"), *of = v.find("data_offsets");
        if (!dt || dt->type != json::Value::String || !sh || sh->type != json::Value::Array || !of ||
            of->type != json::Value::Array) {
            f.set(kInvalid, "Invalid tensor entry: " + entry.first + ".");
            return nullptr;
        }
        StTensor t;
        t.name = entry.first;
        t.dtype = dtype_code(dt->text);
        if (!t.dtype) { f.set(kUnsupported, "Unsupported safetensors dtype '" + dt->text + "'."); return nullptr; }
        if (sh->items.size() < 1 || sh->items.size() > 8) { f.set(kInvalid, "Invalid tensor shape."); return nullptr; }
        int64_t elements = 1;
        for (const auto &d : sh->items) {
            if (!d.is_int32() || d.integer < 1) { f.set(kInvalid, "Invalid tensor shape."); return nullptr; }
            if (elements > INT64_MAX / d.integer) { f.set(kInvalid, "Invalid tensor shape."); return nullptr; }
            elements *= d.integer;
            t.shape.push_back(d.integer);
        }
        if (of->items.size() != 2 || !of->items[0].integral || !of->items[1].integral) {
            f.set(kInvalid, "Invalid tensor offsets/byte length.");
            return nullptr;
        }
        const int64_t o0 = of->items[0].integer, o1 = of->items[1].integer;
        const int eb = dtype_bytes(t.dtype);
        if (o0 < 0 || o1 < o0 || o1 > data_bytes || elements > INT64_MAX / eb || o1 - o0 != elements * eb ||
            elements > INT32_MAX) {
            f.set(kInvalid, "Invalid tensor offsets/byte length.");
            return nullptr;
        }
        t.start = s->data_start + o0;
        t.bytes = o1 - o0;
        if (!s->by_name.emplace(t.name, s->tensors.size()).second) { f.set(kInvalid, "Duplicate tensor name."); return nullptr; }
        s->tensors.push_back(std::move(t));
    }
    std::vector<const StTensor *> order;
    for (const auto &t : s->tensors) order.push_back(&t);
    std::stable_sort(order.begin(), order.end(), [](const StTensor *a, const StTensor *b) { return a->start < b->start; });
    int64_t previous_end = s->data_start;
    for (const StTensor *t : order) {
        if (t->start < previous_end) { f.set(kInvalid, "Overlapping tensors."); return nullptr; }
        previous_end = t->start + t->bytes;
    }
    return s.release();
}

// SafeTensors.Get (SafeTensors.cs:45-50)
const StTensor *st_get(const StFile *s, const std::string &name, const int64_t *shape, int rank, Failure &f) {
    auto it = s->by_name.find(name);
    const StTensor *t = it == s->by_name.end() ? nullptr : &s->tensors[it->second];
    bool same = t && (int)t->shape.size() == rank;
    for (int i = 0; same && i < rank; i++) same = t->shape[i] == shape[i];
    if (!same) {
        f.set(kInvalid, "Missing tensor or shape mismatch: " + name + ".");
        return nullptr;
    }
    return t;
}

StFile *as_st(void *p) {
    StFile *s = static_cast<StFile *>(p);
    return s && s->magic == 0x44495354u ? s : nullptr;
}

const StTensor *st_by_name(const StFile *s, const char *name, Failure &f) {
    auto it = name ? s->by_name.find(name) : s->by_name.end();
    if (it == s->by_name.end()) {
        f.set(kInvalid, std::string("Missing tensor or shape mismatch: ") + (name ? name : "") + ".");
        return nullptr;
    }
    return &s->tensors[it->second];
}

// ReadFloat (SafeTensors.cs:66-82): F32 as is, BF16 widened; any non-finite value rejects
bool st_read_float(const StFile *s, const StTensor *t, float *out, uint64_t count, Failure &f) {
    if (t->dtype != kF32 && t->dtype != kBF16) return f.set(kInvalid, "BF16 tensor required.");
    const uint64_t n = (uint64_t)t->bytes / (uint64_t)dtype_bytes(t->dtype);
    if (count != n) return f.set(kInvalid, "Tensor ownership or destination length mismatch.");
    if (t->dtype == kF32) {
        if (!read_all(s->fd, out, (size_t)t->bytes, t->start)) return f.set(kInvalid, "Tensor read failed.");
    } else {
        std::vector<uint16_t> raw((size_t)n);
        if (!read_all(s->fd, raw.data(), (size_t)t->bytes, t->start)) return f.set(kInvalid, "Tensor read failed.");
        for (uint64_t i = 0; i < n; i++) {
            const uint32_t u = (uint32_t)raw[i] << 16;
            memcpy(&out[i], &u, 4);
        }
    }
    for (uint64_t i = 0; i < n; i++)
        if (!std::isfinite(out[i])) return f.set(kInvalid, "Non-finite tensor values.");
    return true;
}

// ------------------------------------------------------------------------------ checkpoint

constexpr int kDim = 2048, kLayers = 40, kExperts = 256, kSelected = 8, kInter = 512, kVocab = 248320;
constexpr size_t kStageBytes = (size_t)64 << 20;

struct Checkpoint {
    uint32_t magic = 0x4449434bu;
    std::string dir;
    int bits = 0;
    float epsilon = 0.f, rope_theta = 0.f;
    json::Value quant;                                 // config "quantization" object
    std::unordered_map<std::string, std::string> map;  // tensor -> shard file name
    std::unordered_map<std::string, std::unique_ptr<StFile>> shards;
    // upload staging (lazy; on the device of the first context that loads through it)
    int device = -1;
    hipStream_t stream = nullptr;
    void *stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    ~Checkpoint() {
        if (stream) (void)hipStreamSynchronize(stream);
        for (int i = 0; i < 2; i++) {
            if (stage[i]) (void)hipHostFree(stage[i]);
            if (done[i]) (void)hipEventDestroy(done[i]);
        }
        if (stream) (void)hipStreamDestroy(stream);
        magic = 0;
    }
};

Checkpoint *as_ck(void *p) {
    Checkpoint *c = static_cast<Checkpoint *>(p);
    return c && c->magic == 0x4449434bu ? c : nullptr;
}

bool read_text(const std::string &path, std::string &out) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return false;
    struct stat st;
    bool ok = fstat(fd, &st) == 0 && st.st_size >= 0 && st.st_size < ((int64_t)1 << 30);
    if (ok) {
        out.assign((size_t)st.st_size, '\0');
        ok = read_all(fd, out.empty() ? nullptr : &out[0], out.size(), 0);
    }
    ::close(fd);
    return ok;
}

bool get_int(const json::Value &o, const char *key, int64_t &v) {
    const json::Value *x = o.find(key);
    if (!x || !x->is_int32()) return false;
    v = x->integer;
    return true;
}

// Qwen36Weights constructor checks (Qwen36Weights.cs:27-53)
bool ck_config(Checkpoint &c, Failure &f) {
    std::string text, err;
    if (!read_text(c.dir + "/config.json", text)) return f.set(kInvalid, "Cannot read config.json.");
    json::Value root;
    if (!json::parse(text.data(), text.size(), root, err)) return f.set(kInvalid, err + ".");
    const json::Value *mt = root.find("model_type"), *tc = root.find("text_config");
    if (!tc || tc->type != json::Value::Object) return f.set(kUnsupported, "Only the Qwen3.6-35B-A3B text geometry is implemented.");
    struct Want { const char *key; int64_t value; };
    const Want want[] = {{"hidden_size", kDim}, {"num_hidden_layers", kLayers}, {"num_experts", kExperts},
                         {"num_experts_per_tok", kSelected}, {"moe_intermediate_size", kInter},
                         {"vocab_size", kVocab}, {"num_attention_heads", 16}, {"num_key_value_heads", 2},
                         {"head_dim", 256}, {"full_attention_interval", 4}, {"linear_num_value_heads", 32},
                         {"linear_num_key_heads", 16}, {"linear_key_head_dim", 128},
                         {"linear_value_head_dim", 128}, {"linear_conv_kernel_dim", 4}};
    bool ok = mt && mt->type == json::Value::String && mt->text == "qwen3_5_moe";
    for (const Want &w : want) {
        int64_t v;
        ok = ok && get_int(*tc, w.key, v) && v == w.value;
    }
    const json::Value *ntp = tc->find("norm_topk_prob");
    if (ntp && !(ntp->type == json::Value::Bool && ntp->boolean)) ok = false;
    if (!ok) return f.set(kUnsupported, "Only the Qwen3.6-35B-A3B text geometry is implemented.");
    const json::Value *rope = tc->find("rope_parameters");
    int64_t ctx_len;
    if (!get_int(*tc, "max_position_embeddings", ctx_len) || ctx_len != 262144)
        return f.set(kUnsupported, "Expected the pinned 262144-token context geometry.");
    const json::Value *prf = rope ? rope->find("partial_rotary_factor") : nullptr;
    const json::Value *rt = rope ? rope->find("rope_type") : nullptr;
    if (!prf || prf->type != json::Value::Number || (float)prf->number != .25f ||
        (rt && !(rt->type == json::Value::String && rt->text == "default")))
        return f.set(kUnsupported, "Only unscaled text RoPE is implemented; no YaRN/multimodal input.");
    const json::Value *eps = tc->find("rms_norm_eps"), *theta = rope->find("rope_theta");
    if (!eps || eps->type != json::Value::Number || !theta || theta->type != json::Value::Number)
        return f.set(kInvalid, "Invalid Qwen3.6 normalization/RoPE parameters.");
    c.epsilon = (float)eps->number;
    c.rope_theta = (float)theta->number;
    if (!std::isfinite(c.epsilon) || c.epsilon <= 0 || !std::isfinite(c.rope_theta) || c.rope_theta <= 1)
        return f.set(kInvalid, "Invalid Qwen3.6 normalization/RoPE parameters.");
    const json::Value *q = root.find("quantization");
    int64_t bits, group;
    const json::Value *mode = q ? q->find("mode") : nullptr;
    if (!q || !get_int(*q, "bits", bits) || !get_int(*q, "group_size", group) || group != 64 ||
        (bits != 5 && bits != 8) || !mode || mode->type != json::Value::String || mode->text != "affine")
        return f.set(kUnsupported, "Expected affine 5-bit or 8-bit/group64 weights.");
    c.bits = (int)bits;
    c.quant = *q;
    // shard index (Qwen36Weights.cs:54-65)
    if (!read_text(c.dir + "/model.safetensors.index.json", text)) return f.set(kInvalid, "Cannot read model.safetensors.index.json.");
    json::Value index;
    if (!json::parse(text.data(), text.size(), index, err)) return f.set(kInvalid, err + ".");
    const json::Value *wm = index.find("weight_map");
    if (!wm || wm->type != json::Value::Object) return f.set(kInvalid, "Missing weight_map.");
    for (const auto &m : wm->members)
        if (m.second.type == json::Value::String) c.map.emplace(m.first, m.second.text);
    return true;
}

// FileFor (Qwen36Weights.cs:57-64)
StFile *ck_file(Checkpoint &c, const std::string &name, Failure &f) {
    auto it = c.map.find(name);
    if (it == c.map.end()) { f.set(kInvalid, "Missing tensor shard."); return nullptr; }
    const std::string &file = it->second;
    if (file.empty() || file.find('/') != std::string::npos || file.find('\\') != std::string::npos || file == "." ||
        file == "..") {
        f.set(kInvalid, "Unsafe shard path.");
        return nullptr;
    }
    auto sh = c.shards.find(file);
    if (sh != c.shards.end()) return sh->second.get();
    StFile *s = st_open((c.dir + "/" + file).c_str(), f);
    if (!s) return nullptr;
    c.shards.emplace(file, std::unique_ptr<StFile>(s));
    return s;
}

// tensor bytes -> device memory through the two pinned staging buffers
bool ck_upload(Checkpoint &c, int device, const StFile *s, const StTensor *t, void *dst, Failure &f) {
    char e[256];
    if (c.device != device) {
        if (c.device >= 0) return f.set(kInvalid, "One checkpoint loads onto one device.");
        if (!hip_ok(hipSetDevice(device), e, sizeof(e), "set device") ||
            !hip_ok(hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking), e, sizeof(e), "stream") ||
            !hip_ok(hipEventCreateWithFlags(&c.done[0], hipEventDisableTiming), e, sizeof(e), "event") ||
            !hip_ok(hipEventCreateWithFlags(&c.done[1], hipEventDisableTiming), e, sizeof(e), "event") ||
            !hip_ok(hipHostMalloc(&c.stage[0], kStageBytes, hipHostMallocDefault), e, sizeof(e), "pinned staging") ||
            !hip_ok(hipHostMalloc(&c.stage[1], kStageBytes, hipHostMallocDefault), e, sizeof(e), "pinned staging"))
            return f.set(kInvalid, e);
        c.device = device;
        (void)hipEventRecord(c.done[0], c.stream);
        (void)hipEventRecord(c.done[1], c.stream);
    }
    (void)hipSetDevice(device);
    int64_t off = 0;
    for (int k = 0; off < t->bytes; k ^= 1) {
        const size_t n = (size_t)std::min<int64_t>((int64_t)kStageBytes, t->bytes - off);
        if (!hip_ok(hipEventSynchronize(c.done[k]), e, sizeof(e), "staging wait")) return f.set(kInvalid, e);
        if (!read_parallel(s->fd, c.stage[k], n, t->start + off)) return f.set(kInvalid, "Tensor read failed.");
        if (!hip_ok(hipMemcpyAsync(static_cast<char *>(dst) + off, c.stage[k], n, hipMemcpyHostToDevice, c.stream), e,
                    sizeof(e), "weight upload") ||
            !hip_ok(hipEventRecord(c.done[k], c.stream), e, sizeof(e), "staging record"))
            return f.set(kInvalid, e);
        off += (int64_t)n;
    }
    if (!hip_ok(hipStreamSynchronize(c.stream), e, sizeof(e), "weight upload")) return f.set(kInvalid, e);
    return true;
}

// Matrix(prefix, rows, columns, experts, bits) (Qwen36Weights.cs:66-81)
Matrix *ck_matrix(Checkpoint &c, Context *ctx, const std::string &prefix, int rows, int columns, int experts, int bits,
                  Failure &f) {
    bits = bits == 0 ? c.bits : bits;
    if (rows < 1 || columns < 64 || columns % 64 || experts < 1 || (bits != 5 && bits != 8)) {
        f.set(kInvalid, "Invalid matrix geometry: " + prefix);
        return nullptr;
    }
    if (const json::Value *local = c.quant.find(prefix)) {
        int64_t lb, lg;
        const json::Value *mode = local->find("mode");
        if (!get_int(*local, "bits", lb) || lb != bits || !get_int(*local, "group_size", lg) || lg != 64 ||
            (mode && !(mode->type == json::Value::String && mode->text == "affine"))) {
            f.set(kUnsupported, "Unsupported quantization override: " + prefix);
            return nullptr;
        }
    }
    auto shape = [&](int64_t width, int64_t *out) {
        int r = 0;
        if (experts != 1) out[r++] = experts;
        out[r++] = rows;
        out[r++] = width;
        return r;
    };
    int64_t sw[3], ss[3];
    const int rw = shape((int64_t)columns * bits / 32, sw), rs = shape(columns / 64, ss);
    const std::string names[3] = {prefix + ".weight", prefix + ".scales", prefix + ".biases"};
    StFile *files[3];
    const StTensor *ts[3];
    for (int i = 0; i < 3; i++) {
        files[i] = ck_file(c, names[i], f);
        if (!files[i]) return nullptr;
        ts[i] = i == 0 ? st_get(files[i], names[i], sw, rw, f) : st_get(files[i], names[i], ss, rs, f);
        if (!ts[i]) return nullptr;
    }
    if (ts[0]->dtype != kU32 || ts[1]->dtype != kBF16 || ts[2]->dtype != kBF16) {
        f.set(kUnsupported, "Expected U32 packed weights and BF16 affine parameters.");
        return nullptr;
    }
    char e[2048] = {0};
    Matrix *m = static_cast<Matrix *>(dih_quant_matrix_create(ctx, experts, rows, columns, bits, 64, e, sizeof(e)));
    if (!m) {
        f.set(kInvalid, e);
        return nullptr;
    }
    for (int i = 0; i < 3; i++) {
        if ((uint64_t)ts[i]->bytes != m->bytes[i]) {
            dih_quant_matrix_destroy(m);
            f.set(kInvalid, "Tensor ownership or destination length mismatch.");
            return nullptr;
        }
        if (!ck_upload(c, ctx->device, files[i], ts[i], m->dev[i], f)) {
            dih_quant_matrix_destroy(m);
            return nullptr;
        }
    }
    if (!matrix_retile(m, 0, (size_t)m->experts * m->rows, e, sizeof(e))) {
        dih_quant_matrix_destroy(m);
        f.set(kInvalid, e);
        return nullptr;
    }
    return m;
}

void put_status(int *status, int code) {
    if (status) *status = code;
}

}  // namespace

}  // namespace dih

using namespace dih;

extern "C" {

__attribute__((visibility("default"))) void *dih_safetensors_open(const char *path, int *status, char *error,
                                                                  int capacity) {
    Failure f;
    StFile *s = path ? st_open(path, f) : (f.set(kInvalid, "Invalid path."), nullptr);
    put_status(status, s ? kOk : f.code);
    if (!s) set_error(error, capacity, f.message);
    return s;
}

__attribute__((visibility("default"))) void dih_safetensors_close(void *file) { delete as_st(file); }

__attribute__((visibility("default"))) int dih_safetensors_count(void *file) {
    StFile *s = as_st(file);
    return s ? (int)s->tensors.size() : -1;
}

__attribute__((visibility("default"))) int dih_safetensors_info(void *file, int index, char *name, int name_capacity,
                                                                 int *dtype, int *rank, int64_t *shape,
                                                                 uint64_t *bytes) {
    StFile *s = as_st(file);
    if (!s || index < 0 || index >= (int)s->tensors.size()) return -1;
    const StTensor &t = s->tensors[(size_t)index];
    if (name && name_capacity > 0) {
        if ((int)t.name.size() >= name_capacity) return -1;
        memcpy(name, t.name.c_str(), t.name.size() + 1);
    }
    if (dtype) *dtype = t.dtype;
    if (rank) *rank = (int)t.shape.size();
    if (shape)
        for (size_t i = 0; i < t.shape.size(); i++) shape[i] = t.shape[i];
    if (bytes) *bytes = (uint64_t)t.bytes;
    return 0;
}

__attribute__((visibility("default"))) int dih_safetensors_get(void *file, const char *name, const int64_t *shape,
                                                                int rank, char *error, int capacity) {
    StFile *s = as_st(file);
    Failure f;
    if (!s || !name || rank < 0 || rank > 8 || (rank && !shape)) {
        set_error(error, capacity, "Invalid safetensors lookup");
        return kInvalid;
    }
    if (!st_get(s, name, shape, rank, f)) {
        set_error(error, capacity, f.message);
        return f.code;
    }
    return kOk;
}

__attribute__((visibility("default"))) int dih_safetensors_read(void *file, const char *name, int dtype,
                                                                 void *destination, uint64_t bytes, char *error,
                                                                 int capacity) {
    StFile *s = as_st(file);
    Failure f;
    if (!s || !destination) {
        set_error(error, capacity, "Invalid safetensors read");
        return kInvalid;
    }
    const StTensor *t = st_by_name(s, name, f);
    if (t && dtype == kBF16 && t->dtype != kBF16) {
        f.set(kInvalid, "BF16 tensor required.");
        t = nullptr;
    } else if (t && bytes != (uint64_t)t->bytes) {
        f.set(kInvalid, "Tensor ownership or destination length mismatch.");
        t = nullptr;
    } else if (t && !read_all(s->fd, destination, (size_t)t->bytes, t->start)) {
        f.set(kInvalid, "Tensor read failed.");
        t = nullptr;
    }
    if (!t) {
        set_error(error, capacity, f.message);
        return f.code;
    }
    return kOk;
}

__attribute__((visibility("default"))) int dih_safetensors_read_float(void *file, const char *name, float *destination,
                                                                       uint64_t count, char *error, int capacity) {
    StFile *s = as_st(file);
    Failure f;
    if (!s || !destination) {
        set_error(error, capacity, "Invalid safetensors read");
        return kInvalid;
    }
    const StTensor *t = st_by_name(s, name, f);
    if (!t || !st_read_float(s, t, destination, count, f)) {
        set_error(error, capacity, f.message);
        return f.code;
    }
    return kOk;
}

__attribute__((visibility("default"))) void *dih_checkpoint_open(const char *directory, int *status, char *error,
                                                                  int capacity) {
    Failure f;
    std::unique_ptr<Checkpoint> c(new (std::nothrow) Checkpoint());
    if (!c || !directory) {
        put_status(status, kInvalid);
        set_error(error, capacity, "Invalid checkpoint directory");
        return nullptr;
    }
    char resolved[4096];
    c->dir = realpath(directory, resolved) ? resolved : directory;
    if (!ck_config(*c, f)) {
        put_status(status, f.code);
        set_error(error, capacity, f.message);
        return nullptr;
    }
    put_status(status, kOk);
    return c.release();
}

__attribute__((visibility("default"))) void dih_checkpoint_close(void *checkpoint) { delete as_ck(checkpoint); }

__attribute__((visibility("default"))) int dih_checkpoint_info(void *checkpoint, int *bits, float *epsilon,
                                                                float *rope_theta) {
    Checkpoint *c = as_ck(checkpoint);
    if (!c) return -1;
    if (bits) *bits = c->bits;
    if (epsilon) *epsilon = c->epsilon;
    if (rope_theta) *rope_theta = c->rope_theta;
    return 0;
}

__attribute__((visibility("default"))) void *dih_checkpoint_matrix(void *checkpoint, void *context, const char *prefix,
                                                                    int rows, int columns, int experts, int bits,
                                                                    int *status, char *error, int capacity) {
    Checkpoint *c = as_ck(checkpoint);
    Context *ctx = static_cast<Context *>(context);
    Failure f;
    Matrix *m = nullptr;
    if (!c || !ctx || ctx->magic != 0x44494358u || !prefix)
        f.set(kInvalid, "Invalid checkpoint matrix arguments");
    else
        m = ck_matrix(*c, ctx, prefix, rows, columns, experts, bits, f);
    put_status(status, m ? kOk : f.code);
    if (!m) set_error(error, capacity, f.message);
    return m;
}

__attribute__((visibility("default"))) int dih_checkpoint_vector(void *checkpoint, const char *name,
                                                                  const int64_t *shape, int rank, float *destination,
                                                                  uint64_t count, char *error, int capacity) {
    Checkpoint *c = as_ck(checkpoint);
    Failure f;
    if (!c || !name || rank < 1 || rank > 8 || !shape || !destination) {
        set_error(error, capacity, "Invalid checkpoint vector arguments");
        return kInvalid;
    }
    StFile *s = ck_file(*c, name, f);
    const StTensor *t = s ? st_get(s, name, shape, rank, f) : nullptr;
    if (!t || !st_read_float(s, t, destination, count, f)) {
        set_error(error, capacity, f.message);
        return f.code;
    }
    return kOk;
}

__attribute__((visibility("default"))) int dih_checkpoint_moe_layer(void *checkpoint, void *context, int layer,
                                                                     dih_moe_layer *out, char *error, int capacity) {
    Checkpoint *c = as_ck(checkpoint);
    Context *ctx = static_cast<Context *>(context);
    if (!c || !ctx || ctx->magic != 0x44494358u || !out || layer < 0 || layer >= kLayers) {
        set_error(error, capacity, "Invalid checkpoint MoE layer arguments");
        return kInvalid;
    }
    // Qwen36Weights.cs:90-99
    const std::string p = "language_model.model.layers." + std::to_string(layer) + ".";
    struct Spec { const char *name; int rows, columns, experts, bits; void **slot; };
    dih_moe_layer L{};
    const Spec specs[] = {
        {"mlp.gate", kExperts, kDim, 1, 8, &L.router},
        {"mlp.switch_mlp.gate_proj", kInter, kDim, kExperts, 0, &L.gate},
        {"mlp.switch_mlp.up_proj", kInter, kDim, kExperts, 0, &L.up},
        {"mlp.switch_mlp.down_proj", kDim, kInter, kExperts, 0, &L.down},
        {"mlp.shared_expert.gate_proj", kInter, kDim, 1, 0, &L.shared_gate},
        {"mlp.shared_expert.up_proj", kInter, kDim, 1, 0, &L.shared_up},
        {"mlp.shared_expert.down_proj", kDim, kInter, 1, 0, &L.shared_down},
        {"mlp.shared_expert_gate", 1, kDim, 1, 8, &L.shared_route},
    };
    Failure f;
    for (const Spec &s : specs) {
        Matrix *m = ck_matrix(*c, ctx, p + s.name, s.rows, s.columns, s.experts, s.bits, f);
        if (!m) {
            for (const Spec &d : specs)
                if (*d.slot) dih_quant_matrix_destroy(*d.slot);
            set_error(error, capacity, f.message);
            return f.code;
        }
        *s.slot = m;
    }
    *out = L;
    return kOk;
}

}  // extern "C"
