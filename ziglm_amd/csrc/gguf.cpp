// GGUF reader and device-table uploader (C-ABI in include/zl_gguf.h).
//
// Reader: accepts and rejects exactly the files ziglm's GGUFFile.parse does
// (src/gguf.zig:242-317) and extracts ModelParams as gguf.zig:399-451 + types.zig:269-285.
// One forward pass over the header with a bounds-checked cursor; metadata values are not
// copied: each entry records where its bytes sit in the mapped file. Tensor names go into
// a hash map (last duplicate wins, as the reference's StringHashMap.put); metadata lookup
// is a linear scan (first duplicate wins, as getMetadata).
//
// Where the reference would panic (integer overflow in safe builds) this reader returns an
// error instead: general.alignment 0 or not a power of two (ZL_GGUF_EALIGNMENT), a tensor
// whose offset + size overflows 64 bits (ZL_GGUF_EOUT_OF_BOUNDS), a negative INT32/INT64
// read as unsigned (getter reports "absent").
//
// Uploader: tensors are copied file -> pinned slot (host threads) -> device (DMA on the
// caller's stream) through a ring of pinned slots, so host copies of chunk k+1.. overlap
// the transfer of chunk k. The ring is created on first use and kept for the process; a
// mutex serialises uploads. This replaces the reference's one pageable copy per tensor
// (cuda_model.zig:24-36), whose runtime staging is serial.
#include <errno.h>
#include <fcntl.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <mutex>
#include <new>
#include <string>
#include <string_view>
#include <thread>
#include <unordered_map>
#include <vector>

#include <hip/hip_runtime_api.h>

#include "../../include/zl_gguf.h"

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF"

struct Kv {
    std::string_view key;
    uint32_t type = 0, array_type = 0;
    uint64_t array_len = 0;
    const uint8_t* data = nullptr;
    uint64_t bytes = 0;
};

struct TensorRec {
    std::string_view name;
    uint32_t type = 0, n_dims = 0;
    uint64_t shape[4] = {1, 1, 1, 1};
    uint64_t offset = 0;
    const uint8_t* data = nullptr;
    uint64_t size = 0;
};

}  // namespace

struct ZlGguf {
    const uint8_t* base = nullptr;
    uint64_t size = 0;
    bool mapped = false;    // munmap on close
    bool owns = false;      // delete[] on close
    uint32_t version = 0;
    uint64_t tensor_count = 0, metadata_count = 0;
    uint64_t alignment = 32, data_offset = 0;
    std::vector<Kv> kv;
    std::vector<TensorRec> tensors;
    std::unordered_map<std::string_view, size_t> by_name;
    ZlModelParams params{};
};

namespace {

// ---- GGML type sizes (types.zig:33-67) ---------------------------------------------
uint64_t block_size(uint32_t t) {
    switch (t) {
        case 0: case 1: case 16: case 17: case 18: case 19: case 20: case 30:  // F32 F16 I8 I16 I32 I64 F64 BF16
            return 1;
        case 10: case 11: case 12: case 13: case 14: case 15:  // Q2_K .. Q8_K
        case 21: case 23: case 24: case 25:                     // IQ1_S IQ3_S IQ2_S IQ4_XS
            return 256;
        default:  // Q4_0 Q4_1 Q5_0 Q5_1 Q8_0 Q8_1 IQ4_NL and everything else
            return 32;
    }
}

uint64_t type_size(uint32_t t) {
    switch (t) {
        case 0: return 4;     // F32
        case 1: return 2;     // F16
        case 30: return 2;    // BF16
        case 16: return 1;    // I8
        case 17: return 2;    // I16
        case 18: return 4;    // I32
        case 19: return 8;    // I64
        case 20: return 8;    // F64
        case 2: return 18;    // Q4_0: f16 d + 16 B of nibbles
        case 3: return 20;    // Q4_1: f16 d, f16 m + 16 B
        case 6: return 22;    // Q5_0: f16 d + 4 B high bits + 16 B
        case 7: return 24;    // Q5_1
        case 8: return 34;    // Q8_0: f16 d + 32 i8
        case 9: return 36;    // Q8_1
        case 10: return 84;   // Q2_K
        case 11: return 110;  // Q3_K
        case 12: return 144;  // Q4_K
        case 13: return 176;  // Q5_K
        case 14: return 210;  // Q6_K
        case 15: return 292;  // Q8_K
        case 22: return 18;   // IQ4_NL
        default: return 1;    // the reference's fallback
    }
}

// Fixed byte size of a scalar value type, 0 for STRING / ARRAY / unknown.
uint64_t scalar_bytes(uint32_t t) {
    switch (t) {
        case ZL_GGUF_UINT8: case ZL_GGUF_INT8: case ZL_GGUF_BOOL: return 1;
        case ZL_GGUF_UINT16: case ZL_GGUF_INT16: return 2;
        case ZL_GGUF_UINT32: case ZL_GGUF_INT32: case ZL_GGUF_FLOAT32: return 4;
        case ZL_GGUF_UINT64: case ZL_GGUF_INT64: case ZL_GGUF_FLOAT64: return 8;
        default: return 0;
    }
}

template <typename T> T load_le(const uint8_t* p) {
    T v;
    memcpy(&v, p, sizeof(T));  // x86-64 and gfx hosts are little endian
    return v;
}

struct Cursor {
    const uint8_t* base;
    uint64_t size, pos = 0;
    int err = 0;

    bool need(uint64_t n) {
        if (err) return false;
        if (n > size - pos) {
            err = ZL_GGUF_EEOF;
            return false;
        }
        return true;
    }
    template <typename T> T get() {
        if (!need(sizeof(T))) return T{};
        T v = load_le<T>(base + pos);
        pos += sizeof(T);
        return v;
    }
    std::string_view str() {
        const uint64_t n = get<uint64_t>();
        if (!need(n)) return {};
        std::string_view s(reinterpret_cast<const char*>(base + pos), n);
        pos += n;
        return s;
    }
    // Skip one value of type t (gguf.zig:213-239 parseValue); arrays recurse per element.
    void skip_value(uint32_t t) {
        if (err) return;
        if (const uint64_t b = scalar_bytes(t)) {
            if (need(b)) pos += b;
            return;
        }
        if (t == ZL_GGUF_STRING) {
            str();
            return;
        }
        if (t == ZL_GGUF_ARRAY) {
            const uint32_t et = get<uint32_t>();
            const uint64_t n = get<uint64_t>();
            if (err || n == 0) return;  // an empty array of any type is accepted
            if (const uint64_t b = scalar_bytes(et)) {
                if (n > (size - pos) / b) {
                    err = ZL_GGUF_EEOF;
                    return;
                }
                pos += n * b;
                return;
            }
            if (et != ZL_GGUF_STRING && et != ZL_GGUF_ARRAY) {
                err = ZL_GGUF_EVALUE_TYPE;
                return;
            }
            for (uint64_t i = 0; i < n && !err; ++i) skip_value(et);
            return;
        }
        err = ZL_GGUF_EVALUE_TYPE;
    }
};

int parse(ZlGguf* f) {
    Cursor c{f->base, f->size};
    if (c.get<uint32_t>() != kMagic) return c.err ? c.err : ZL_GGUF_EMAGIC;
    f->version = c.get<uint32_t>();
    if (c.err) return c.err;
    if (f->version != 2 && f->version != 3) return ZL_GGUF_EVERSION;
    f->tensor_count = c.get<uint64_t>();
    f->metadata_count = c.get<uint64_t>();
    if (c.err) return c.err;

    // An entry takes at least 13 bytes (key length, type, one byte of value): never reserve
    // more than the file can hold.
    f->kv.reserve(std::min<uint64_t>(f->metadata_count, (f->size - c.pos) / 13 + 1));
    for (uint64_t i = 0; i < f->metadata_count; ++i) {
        Kv e;
        e.key = c.str();
        e.type = c.get<uint32_t>();
        if (c.err) return c.err;
        const uint64_t start = c.pos;
        if (e.type == ZL_GGUF_ARRAY) {
            e.array_type = c.get<uint32_t>();
            e.array_len = c.get<uint64_t>();
            if (c.err) return c.err;
            const uint64_t elems = c.pos;
            c.pos = start;
            c.skip_value(ZL_GGUF_ARRAY);
            if (c.err) return c.err;
            e.data = f->base + elems;
            e.bytes = c.pos - elems;
        } else if (e.type == ZL_GGUF_STRING) {
            std::string_view s = c.str();
            if (c.err) return c.err;
            e.data = reinterpret_cast<const uint8_t*>(s.data());
            e.bytes = s.size();
        } else {
            c.skip_value(e.type);
            if (c.err) return c.err;
            e.data = f->base + start;
            e.bytes = c.pos - start;
        }
        // gguf.zig:264-266: only a UINT32 value sets the alignment
        if (e.key == "general.alignment" && e.type == ZL_GGUF_UINT32)
            f->alignment = load_le<uint32_t>(e.data);
        f->kv.push_back(e);
    }

    f->tensors.reserve(std::min<uint64_t>(f->tensor_count, (f->size - c.pos) / 24 + 1));
    for (uint64_t i = 0; i < f->tensor_count; ++i) {
        TensorRec t;
        t.name = c.str();
        t.n_dims = c.get<uint32_t>();
        if (c.err) return c.err;
        if (t.n_dims > 4) return ZL_GGUF_EDIMS;
        for (uint32_t d = 0; d < t.n_dims; ++d) t.shape[d] = c.get<uint64_t>();
        t.type = c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        if (c.err) return c.err;
        f->by_name[t.name] = f->tensors.size();
        f->tensors.push_back(t);
    }

    const uint64_t a = f->alignment;
    if (a == 0 || (a & (a - 1))) return ZL_GGUF_EALIGNMENT;
    if (c.pos > UINT64_MAX - (a - 1)) return ZL_GGUF_EOUT_OF_BOUNDS;
    f->data_offset = (c.pos + a - 1) & ~(a - 1);

    for (TensorRec& t : f->tensors) {
        uint64_t elems = 1;
        for (uint32_t d = 0; d < t.n_dims; ++d) elems *= t.shape[d];  // wraps like usize math
        t.size = elems / block_size(t.type) * type_size(t.type);
        const uint64_t abs = f->data_offset + t.offset;
        if (abs < t.offset || abs + t.size < abs || abs + t.size > f->size) return ZL_GGUF_EOUT_OF_BOUNDS;
        t.data = f->base + abs;
    }
    return 0;
}

// ---- getters (gguf.zig:326-389) ----------------------------------------------------
const Kv* find_kv(const ZlGguf* f, std::string_view key) {
    for (const Kv& e : f->kv)
        if (e.key == key) return &e;
    return nullptr;
}

bool get_u64(const ZlGguf* f, std::string_view key, uint64_t* out) {
    const Kv* e = find_kv(f, key);
    if (!e) return false;
    auto from = [&](uint32_t t, const uint8_t* p) -> bool {
        switch (t) {
            case ZL_GGUF_UINT64: *out = load_le<uint64_t>(p); return true;
            case ZL_GGUF_UINT32: *out = load_le<uint32_t>(p); return true;
            case ZL_GGUF_INT64: {
                const int64_t v = load_le<int64_t>(p);
                if (v < 0) return false;
                *out = (uint64_t)v;
                return true;
            }
            case ZL_GGUF_INT32: {
                const int32_t v = load_le<int32_t>(p);
                if (v < 0) return false;
                *out = (uint64_t)v;
                return true;
            }
            default: return false;
        }
    };
    if (e->type == ZL_GGUF_ARRAY) {
        if (e->array_len == 0) return false;
        const uint64_t b = scalar_bytes(e->array_type);
        if (b == 0 || e->bytes < b) return false;
        return from(e->array_type, e->data);
    }
    return from(e->type, e->data);
}

bool get_u32(const ZlGguf* f, std::string_view key, uint32_t* out) {
    const Kv* e = find_kv(f, key);
    if (!e) return false;
    switch (e->type) {
        case ZL_GGUF_UINT32: *out = load_le<uint32_t>(e->data); return true;
        case ZL_GGUF_UINT64: *out = (uint32_t)load_le<uint64_t>(e->data); return true;  // truncated
        case ZL_GGUF_INT32: {
            const int32_t v = load_le<int32_t>(e->data);
            if (v < 0) return false;
            *out = (uint32_t)v;
            return true;
        }
        default: return false;
    }
}

bool get_f32(const ZlGguf* f, std::string_view key, float* out) {
    const Kv* e = find_kv(f, key);
    if (!e) return false;
    switch (e->type) {
        case ZL_GGUF_FLOAT32: *out = load_le<float>(e->data); return true;
        case ZL_GGUF_FLOAT64: *out = (float)load_le<double>(e->data); return true;
        case ZL_GGUF_ARRAY:
            if (e->array_len > 0 && e->array_type == ZL_GGUF_FLOAT32 && e->bytes >= 4) {
                *out = load_le<float>(e->data);
                return true;
            }
            return false;
        default: return false;
    }
}

bool get_string(const ZlGguf* f, std::string_view key, std::string_view* out) {
    const Kv* e = find_kv(f, key);
    if (!e || e->type != ZL_GGUF_STRING) return false;
    *out = std::string_view(reinterpret_cast<const char*>(e->data), e->bytes);
    return true;
}

// ---- parameters (gguf.zig:399-451, types.zig:225-238, 246-285) ---------------------
int32_t arch_of(std::string_view s) {
    if (s == "llama") return ZL_ARCH_LLAMA;
    if (s == "qwen2" || s == "qwen2.5") return ZL_ARCH_QWEN2;
    if (s == "mistral") return ZL_ARCH_MISTRAL;
    if (s == "gemma") return ZL_ARCH_GEMMA;
    if (s == "gemma2") return ZL_ARCH_GEMMA2;
    if (s == "gemma4" || s == "gemma_4") return ZL_ARCH_GEMMA4;
    if (s == "phi" || s == "phi2") return ZL_ARCH_PHI;
    if (s == "phi3") return ZL_ARCH_PHI3;
    if (s == "deepseek") return ZL_ARCH_DEEPSEEK;
    if (s == "starcoder2") return ZL_ARCH_STARCODER2;
    if (s == "gpt2") return ZL_ARCH_GPT2;
    return ZL_ARCH_UNKNOWN;
}

void extract_params(const ZlGguf* f, ZlModelParams* p) {
    // ModelParams defaults (types.zig:247-267)
    *p = ZlModelParams{};
    p->arch = ZL_ARCH_LLAMA;
    p->context_length = 2048;
    p->embedding_length = 4096;
    p->feed_forward_length = 11008;
    p->head_count = 32;
    p->head_count_kv = 32;
    p->block_count = 32;
    p->vocab_size = 32000;
    p->layer_norm_rms_epsilon = 1e-5f;
    p->rope_freq_base = 10000.0f;
    p->rope_freq_scale = 1.0f;

    std::string_view arch = "llama";
    get_string(f, "general.architecture", &arch);
    p->arch = arch_of(arch);
    // "{arch}.{name}" is formatted into a 128-byte buffer; a longer key is never found
    auto key = [&](const char* name, std::string* out) {
        *out = std::string(arch) + "." + name;
        return out->size() <= 128;
    };
    std::string k;
    auto u64 = [&](const char* name, uint64_t* dst) {
        uint64_t v;
        if (key(name, &k) && get_u64(f, k, &v)) {
            *dst = v;
            return true;
        }
        return false;
    };
    auto f32 = [&](const char* name, float* dst) {
        float v;
        if (key(name, &k) && get_f32(f, k, &v)) *dst = v;
    };
    u64("context_length", &p->context_length);
    u64("embedding_length", &p->embedding_length);
    u64("feed_forward_length", &p->feed_forward_length);
    u64("block_count", &p->block_count);
    u64("attention.head_count", &p->head_count);
    if (!u64("attention.head_count_kv", &p->head_count_kv)) p->head_count_kv = p->head_count;
    u64("attention.key_length", &p->head_size);
    u64("attention.sliding_window", &p->sliding_window);
    f32("attention.layer_norm_rms_epsilon", &p->layer_norm_rms_epsilon);
    f32("rope.freq_base", &p->rope_freq_base);
    f32("rope.freq_scale", &p->rope_freq_scale);
    u64("rope.dimension_count", &p->rope_dim_count);
    f32("final_logit_softcapping", &p->final_logit_softcapping);
    auto it = f->by_name.find("token_embd.weight");
    if (it != f->by_name.end()) p->vocab_size = f->tensors[it->second].shape[1];

    // initComputed (types.zig:269-285)
    if (p->head_count > 0 && p->head_size == 0) p->head_size = p->embedding_length / p->head_count;
    if (p->rope_dim_count == 0) p->rope_dim_count = p->head_size;
    if (p->head_count_kv == 0) p->head_count_kv = p->head_count;
    if (p->arch == ZL_ARCH_GEMMA || p->arch == ZL_ARCH_GEMMA2) p->use_gemma_rms_unit_offset = 1;
    else if (p->arch == ZL_ARCH_GEMMA4) p->use_gemma_rms_unit_offset = 0;
}

int finish_open(ZlGguf* f, ZlGguf** out) {
    const int rc = parse(f);
    if (rc != 0) {
        zl_gguf_close(f);
        return rc;
    }
    extract_params(f, &f->params);
    *out = f;
    return 0;
}

// ---- pinned ring uploader ------------------------------------------------------------
constexpr int kSlots = 4;
constexpr uint64_t kSlotBytes = 16ull << 20;
constexpr uint64_t kThreadMin = 1ull << 20;  // split host copies above this size
constexpr int kMaxThreads = 8;

struct Ring {
    uint8_t* slot[kSlots] = {};
    hipEvent_t done[kSlots] = {};
    bool busy[kSlots] = {};
    int next = 0;
    bool ready = false;
};

std::mutex g_ring_mu;
Ring g_ring;

int ring_init() {
    if (g_ring.ready) return 0;
    for (int i = 0; i < kSlots; ++i) {
        hipError_t e = hipHostMalloc(reinterpret_cast<void**>(&g_ring.slot[i]), kSlotBytes, hipHostMallocDefault);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&g_ring.done[i], hipEventDisableTiming);
        if (e != hipSuccess) {
            for (int j = 0; j <= i; ++j) {
                if (g_ring.slot[j]) (void)hipHostFree(g_ring.slot[j]);
                if (g_ring.done[j]) (void)hipEventDestroy(g_ring.done[j]);
                g_ring.slot[j] = nullptr;
                g_ring.done[j] = nullptr;
            }
            return (int)e;
        }
    }
    g_ring.ready = true;
    return 0;
}

void host_copy(uint8_t* dst, const uint8_t* src, uint64_t n) {
    const int hw = (int)std::max(1u, std::thread::hardware_concurrency());
    const int t = (int)std::min<uint64_t>(std::min(kMaxThreads, hw), std::max<uint64_t>(1, n / kThreadMin));
    if (t <= 1) {
        memcpy(dst, src, n);
        return;
    }
    const uint64_t part = (n / t + 4095) & ~4095ull;  // page-sized pieces
    std::vector<std::thread> pool;
    pool.reserve(t - 1);
    for (int i = 1; i < t; ++i) {
        const uint64_t lo = std::min<uint64_t>(n, i * part), hi = std::min<uint64_t>(n, lo + part);
        if (lo < hi) pool.emplace_back([=] { memcpy(dst + lo, src + lo, hi - lo); });
    }
    memcpy(dst, src, std::min(n, part));
    for (std::thread& th : pool) th.join();
}

// Enqueue `n` bytes src -> dst through the ring (caller holds g_ring_mu).
int ring_copy(void* dst, const void* src, uint64_t n, hipStream_t s) {
    auto* d = static_cast<uint8_t*>(dst);
    auto* h = static_cast<const uint8_t*>(src);
    for (uint64_t off = 0; off < n; off += kSlotBytes) {
        const uint64_t len = std::min(kSlotBytes, n - off);
        const int k = g_ring.next;
        g_ring.next = (k + 1) % kSlots;
        if (g_ring.busy[k]) {
            hipError_t e = hipEventSynchronize(g_ring.done[k]);
            if (e != hipSuccess) return (int)e;
        }
        host_copy(g_ring.slot[k], h + off, len);
        hipError_t e = hipMemcpyAsync(d + off, g_ring.slot[k], len, hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipEventRecord(g_ring.done[k], s);
        if (e != hipSuccess) return (int)e;
        g_ring.busy[k] = true;
    }
    return 0;
}

int ring_drain() {
    for (int k = 0; k < kSlots; ++k) {
        if (!g_ring.busy[k]) continue;
        hipError_t e = hipEventSynchronize(g_ring.done[k]);
        if (e != hipSuccess) return (int)e;
        g_ring.busy[k] = false;
    }
    return 0;
}

}  // namespace

extern "C" {

int zl_gguf_open(const char* path, ZlGguf** out) {
    if (!out) return ZL_GGUF_EINVAL;
    *out = nullptr;
    if (!path) return ZL_GGUF_EINVAL;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return ZL_GGUF_EOPEN;
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return ZL_GGUF_EOPEN;
    }
    const uint64_t n = (uint64_t)st.st_size;
    if (n < 24) {
        close(fd);
        return ZL_GGUF_EINVALID_FILE;
    }
    ZlGguf* f = new (std::nothrow) ZlGguf;
    if (!f) {
        close(fd);
        return ZL_GGUF_ENOMEM;
    }
    f->size = n;
    void* m = mmap(nullptr, n, PROT_READ, MAP_SHARED, fd, 0);
    if (m != MAP_FAILED) {
        f->base = static_cast<const uint8_t*>(m);
        f->mapped = true;
    } else {
        // read the whole file instead (gguf.zig:92-104)
        uint8_t* buf = new (std::nothrow) uint8_t[n];
        if (!buf) {
            close(fd);
            delete f;
            return ZL_GGUF_ENOMEM;
        }
        uint64_t got = 0;
        while (got < n) {
            const ssize_t r = read(fd, buf + got, n - got);
            if (r < 0 && errno == EINTR) continue;
            if (r <= 0) break;
            got += (uint64_t)r;
        }
        f->base = buf;
        f->owns = true;
        f->size = got;
    }
    close(fd);
    return finish_open(f, out);
}

int zl_gguf_open_buffer(const void* data, uint64_t size, ZlGguf** out) {
    if (!out) return ZL_GGUF_EINVAL;
    *out = nullptr;
    if (!data && size) return ZL_GGUF_EINVAL;
    ZlGguf* f = new (std::nothrow) ZlGguf;
    if (!f) return ZL_GGUF_ENOMEM;
    f->base = static_cast<const uint8_t*>(data);
    f->size = size;
    return finish_open(f, out);
}

void zl_gguf_close(ZlGguf* f) {
    if (!f) return;
    if (f->mapped) munmap(const_cast<uint8_t*>(f->base), f->size);
    else if (f->owns) delete[] f->base;
    delete f;
}

const char* zl_gguf_error_name(int code) {
    switch (code) {
        case ZL_GGUF_OK: return "OK";
        case ZL_GGUF_EOPEN: return "FileOpenFailed";
        case ZL_GGUF_EINVALID_FILE: return "InvalidGGUFFile";
        case ZL_GGUF_EMAGIC: return "InvalidGGUFMagic";
        case ZL_GGUF_EVERSION: return "UnsupportedGGUFVersion";
        case ZL_GGUF_EEOF: return "UnexpectedEOF";
        case ZL_GGUF_EVALUE_TYPE: return "UnsupportedGGUFValueType";
        case ZL_GGUF_EDIMS: return "InvalidTensorDimensions";
        case ZL_GGUF_EOUT_OF_BOUNDS: return "TensorDataOutOfBounds";
        case ZL_GGUF_EALIGNMENT: return "InvalidAlignment";
        case ZL_GGUF_ENOMEM: return "OutOfMemory";
        case ZL_GGUF_EINVAL: return "InvalidArgument";
        case ZL_GGUF_ESIZE: return "DestinationTooSmall";
        default: return hipGetErrorName((hipError_t)code);
    }
}

uint32_t zl_gguf_version(const ZlGguf* f) { return f ? f->version : 0; }
uint64_t zl_gguf_tensor_count(const ZlGguf* f) { return f ? f->tensor_count : 0; }
uint64_t zl_gguf_metadata_count(const ZlGguf* f) { return f ? f->metadata_count : 0; }
uint64_t zl_gguf_alignment(const ZlGguf* f) { return f ? f->alignment : 0; }
uint64_t zl_gguf_data_offset(const ZlGguf* f) { return f ? f->data_offset : 0; }
uint64_t zl_gguf_file_size(const ZlGguf* f) { return f ? f->size : 0; }
const void* zl_gguf_base(const ZlGguf* f) { return f ? f->base : nullptr; }

int zl_gguf_metadata(const ZlGguf* f, uint64_t index, ZlGgufKV* out) {
    if (!f || !out || index >= f->kv.size()) return ZL_GGUF_EINVAL;
    const Kv& e = f->kv[index];
    out->key = e.key.data();
    out->key_len = e.key.size();
    out->type = e.type;
    out->array_type = e.array_type;
    out->array_len = e.array_len;
    out->data = e.data;
    out->data_bytes = e.bytes;
    return 0;
}

int64_t zl_gguf_find_metadata(const ZlGguf* f, const char* key) {
    if (!f || !key) return -1;
    const Kv* e = find_kv(f, key);
    return e ? (int64_t)(e - f->kv.data()) : -1;
}

int zl_gguf_get_u32(const ZlGguf* f, const char* key, uint32_t* out) {
    return (f && key && out && get_u32(f, key, out)) ? 1 : 0;
}
int zl_gguf_get_u64(const ZlGguf* f, const char* key, uint64_t* out) {
    return (f && key && out && get_u64(f, key, out)) ? 1 : 0;
}
int zl_gguf_get_f32(const ZlGguf* f, const char* key, float* out) {
    return (f && key && out && get_f32(f, key, out)) ? 1 : 0;
}
int zl_gguf_get_string(const ZlGguf* f, const char* key, const char** s, uint64_t* len) {
    std::string_view v;
    if (!f || !key || !s || !len || !get_string(f, key, &v)) return 0;
    *s = v.data();
    *len = v.size();
    return 1;
}

int zl_gguf_tensor(const ZlGguf* f, uint64_t index, ZlGgufTensor* out) {
    if (!f || !out || index >= f->tensors.size()) return ZL_GGUF_EINVAL;
    const TensorRec& t = f->tensors[index];
    out->name = t.name.data();
    out->name_len = t.name.size();
    out->type = t.type;
    out->n_dims = t.n_dims;
    for (int d = 0; d < 4; ++d) out->shape[d] = t.shape[d];
    out->offset = t.offset;
    out->data = t.data;
    out->size_bytes = t.size;
    return 0;
}

int64_t zl_gguf_find_tensor(const ZlGguf* f, const char* name, ZlGgufTensor* out) {
    if (!f || !name) return -1;
    auto it = f->by_name.find(std::string_view(name));
    if (it == f->by_name.end()) return -1;
    if (out) zl_gguf_tensor(f, it->second, out);
    return (int64_t)it->second;
}

uint64_t zl_ggml_block_size(uint32_t type) { return block_size(type); }
uint64_t zl_ggml_type_size(uint32_t type) { return type_size(type); }

void zl_gguf_params(const ZlGguf* f, ZlModelParams* out) {
    if (f && out) *out = f->params;
}

int zl_gguf_upload_tensors(const ZlGguf* f, const uint64_t* indices, void* const* dsts,
                           const uint64_t* dst_bytes, uint64_t n, HipStream_t stream) {
    if (!f || (n && (!indices || !dsts || !dst_bytes))) return ZL_GGUF_EINVAL;
    for (uint64_t i = 0; i < n; ++i) {
        if (indices[i] >= f->tensors.size() || !dsts[i]) return ZL_GGUF_EINVAL;
        if (dst_bytes[i] < f->tensors[indices[i]].size) return ZL_GGUF_ESIZE;
    }
    std::lock_guard<std::mutex> lock(g_ring_mu);
    int rc = ring_init();
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    for (uint64_t i = 0; i < n && rc == 0; ++i) {
        const TensorRec& t = f->tensors[indices[i]];
        rc = ring_copy(dsts[i], t.data, t.size, s);
    }
    const int rd = ring_drain();
    return rc ? rc : rd;
}

int zl_gguf_upload(const ZlGguf* f, uint64_t index, void* dst, uint64_t dst_bytes, HipStream_t stream) {
    return zl_gguf_upload_tensors(f, &index, &dst, &dst_bytes, 1, stream);
}

int zl_upload_host(void* dst, const void* src, uint64_t bytes, HipStream_t stream) {
    if (bytes == 0) return 0;
    if (!dst || !src) return ZL_GGUF_EINVAL;
    std::lock_guard<std::mutex> lock(g_ring_mu);
    int rc = ring_init();
    if (rc == 0) rc = ring_copy(dst, src, bytes, reinterpret_cast<hipStream_t>(stream));
    const int rd = ring_drain();
    return rc ? rc : rd;
}

}  // extern "C"
