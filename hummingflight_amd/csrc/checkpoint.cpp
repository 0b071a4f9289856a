// checkpoint.cpp -- safetensors checkpoints -> registered MoE layers.
//
// The counterpart of the reference's checkpoint index (WeightIndex::build,
// src/model/weight_index.cpp:84-266) and strict shard parser
// (SafeTensorsFile::open, src/model/safetensors.cpp:60-240), reduced to what
// the MoE block needs: find a layer's router, correction bias, shared expert,
// post-attention norm and routed experts, check them, and copy them once into
// HBM (or, for streamed layers, pinned host RAM with each expert laid out as
// [gate | up | down], the scheduler's assembly order, scheduler.cpp:437-471).
//
// Shard format: u64 little-endian header length n, n bytes of JSON
// {name: {dtype, shape, data_offsets: [begin, end]}, "__metadata__": ...},
// then the data area; offsets are relative to its start (8 + n).
// Validation is the reference's strict mode (strictStOpts, weight_index.cpp:
// 20-27): n a multiple of 8, a parseable JSON object, then per tensor a known
// dtype, BF16 only except F32 for names containing "e_score_correction_bias",
// a non-empty shape of non-negative integers, offsets [begin < end] inside the
// file, an 8-byte-aligned absolute data start, shape x dtype size equal to the
// byte span, and no second tensor of one name.  Rejected tensors are counted
// per reason (SafeTensorsStats, safetensors.h:50-61) and left out.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cctype>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <dirent.h>
#include <memory>
#include <set>
#include <thread>

#include "hf_api_internal.h"

namespace hf {
namespace {

// ---- a small JSON reader (objects, arrays, strings, numbers, literals) ----
struct JVal {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    double num = 0.0;
    bool b = false;
    std::string str;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;  // in document order, duplicates kept
    const JVal* get(const char* key) const {
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class JParser {
public:
    JParser(const char* p, size_t n) : p_(p), end_(p + n) {}
    bool parse(JVal& v) {
        if (!value(v, 0)) return false;
        ws();
        return p_ == end_;
    }

private:
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char* s) {
        const size_t n = strlen(s);
        if ((size_t)(end_ - p_) < n || memcmp(p_, s, n) != 0) return false;
        p_ += n;
        return true;
    }
    bool string(std::string& out) {
        if (p_ >= end_ || *p_ != '"') return false;
        ++p_;
        while (p_ < end_ && *p_ != '"') {
            char c = *p_++;
            if (c == '\\') {
                if (p_ >= end_) return false;
                char e = *p_++;
                switch (e) {
                    case '"': case '\\': case '/': out += e; break;
                    case 'b': out += '\b'; break;
                    case 'f': out += '\f'; break;
                    case 'n': out += '\n'; break;
                    case 'r': out += '\r'; break;
                    case 't': out += '\t'; break;
                    case 'u': {
                        if (end_ - p_ < 4) return false;
                        unsigned cp = 0;
                        for (int i = 0; i < 4; ++i) {
                            const char h = *p_++;
                            cp <<= 4;
                            if (h >= '0' && h <= '9') cp |= h - '0';
                            else if (h >= 'a' && h <= 'f') cp |= h - 'a' + 10;
                            else if (h >= 'A' && h <= 'F') cp |= h - 'A' + 10;
                            else return false;
                        }
                        // UTF-8 of a BMP code point (tensor names are ASCII in practice).
                        if (cp < 0x80) out += (char)cp;
                        else if (cp < 0x800) { out += (char)(0xC0 | (cp >> 6)); out += (char)(0x80 | (cp & 0x3F)); }
                        else { out += (char)(0xE0 | (cp >> 12)); out += (char)(0x80 | ((cp >> 6) & 0x3F)); out += (char)(0x80 | (cp & 0x3F)); }
                        break;
                    }
                    default: return false;
                }
            } else if ((unsigned char)c < 0x20) {
                return false;
            } else {
                out += c;
            }
        }
        if (p_ >= end_) return false;
        ++p_;
        return true;
    }
    bool number(double& out) {
        const char* s = p_;
        if (p_ < end_ && *p_ == '-') ++p_;
        if (p_ >= end_ || !isdigit((unsigned char)*p_)) return false;
        while (p_ < end_ && (isdigit((unsigned char)*p_) || *p_ == '.' || *p_ == 'e' || *p_ == 'E' ||
                             *p_ == '+' || *p_ == '-'))
            ++p_;
        std::string tok(s, p_);
        char* e = nullptr;
        out = strtod(tok.c_str(), &e);
        return e && *e == '\0';
    }
    bool value(JVal& v, int depth) {
        if (depth > 64) return false;
        ws();
        if (p_ >= end_) return false;
        const char c = *p_;
        if (c == '{') {
            ++p_;
            v.kind = JVal::OBJ;
            ws();
            if (p_ < end_ && *p_ == '}') { ++p_; return true; }
            for (;;) {
                ws();
                std::string key;
                if (!string(key)) return false;
                ws();
                if (p_ >= end_ || *p_ != ':') return false;
                ++p_;
                JVal child;
                if (!value(child, depth + 1)) return false;
                v.obj.emplace_back(std::move(key), std::move(child));
                ws();
                if (p_ < end_ && *p_ == ',') { ++p_; continue; }
                if (p_ < end_ && *p_ == '}') { ++p_; return true; }
                return false;
            }
        }
        if (c == '[') {
            ++p_;
            v.kind = JVal::ARR;
            ws();
            if (p_ < end_ && *p_ == ']') { ++p_; return true; }
            for (;;) {
                JVal child;
                if (!value(child, depth + 1)) return false;
                v.arr.push_back(std::move(child));
                ws();
                if (p_ < end_ && *p_ == ',') { ++p_; continue; }
                if (p_ < end_ && *p_ == ']') { ++p_; return true; }
                return false;
            }
        }
        if (c == '"') { v.kind = JVal::STR; return string(v.str); }
        if (lit("true")) { v.kind = JVal::BOOL; v.b = true; return true; }
        if (lit("false")) { v.kind = JVal::BOOL; return true; }
        if (lit("null")) { v.kind = JVal::NUL; return true; }
        v.kind = JVal::NUM;
        return number(v.num);
    }
    const char* p_;
    const char* end_;
};

size_t dtype_bytes(const std::string& d) {
    static const std::map<std::string, size_t> k = {
        {"F64", 8}, {"F32", 4}, {"F16", 2}, {"BF16", 2}, {"I64", 8}, {"I32", 4},
        {"I16", 2}, {"I8", 1}, {"U64", 8}, {"U32", 4}, {"U8", 1}, {"BOOL", 1}};
    auto it = k.find(d);
    return it == k.end() ? 0 : it->second;
}

bool ends_with(const std::string& s, const char* suf) {
    const size_t n = strlen(suf);
    return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

}  // namespace

struct Shard {
    std::string path;
    int fd = -1;
    const uint8_t* base = nullptr;  // whole file, read-only mapping
    size_t size = 0;
    uint64_t data0 = 0;             // 8 + header length
    ~Shard() {
        if (base) munmap(const_cast<uint8_t*>(base), size);
        if (fd >= 0) close(fd);
    }
};

struct TensorRef {
    const Shard* shard = nullptr;
    std::string dtype;
    std::vector<int64_t> shape;
    uint64_t begin = 0, end = 0;
    const uint8_t* data() const { return shard->base + shard->data0 + begin; }
    uint64_t bytes() const { return end - begin; }
};

struct LoadedLayer {
    std::vector<void*> dev;   // hipMalloc'd
    std::vector<void*> host;  // hipHostMalloc'd
};

}  // namespace hf

struct hfmoe_checkpoint {
    std::vector<std::unique_ptr<hf::Shard>> shards;
    std::map<std::string, hf::TensorRef> tensors;
    hfmoe_safetensors_stats stats{};
    std::map<int, hf::LoadedLayer> loaded;
    hf::LoadedLayer lm_head;  // lm_head.weight + model.norm.weight
};

namespace hf {
namespace {

// Parses one shard and adds its accepted tensors (those in `wanted`, when
// given) to ck.  Returns false when the shard as a whole is unreadable.
bool open_shard(hfmoe_checkpoint& ck, const std::string& path, const std::map<std::string, std::string>* wanted,
                const std::string& shard_name, std::string& err) {
    auto sh = std::make_unique<Shard>();
    sh->path = path;
    sh->fd = open(path.c_str(), O_RDONLY);
    if (sh->fd < 0) {
        err = "cannot open " + path;
        return false;
    }
    struct stat st;
    if (fstat(sh->fd, &st) != 0 || st.st_size < 8) {
        err = "cannot read the header length of " + path;
        return false;
    }
    sh->size = (size_t)st.st_size;
    void* m = mmap(nullptr, sh->size, PROT_READ, MAP_PRIVATE, sh->fd, 0);
    if (m == MAP_FAILED) {
        err = "mmap failed for " + path;
        return false;
    }
    sh->base = static_cast<const uint8_t*>(m);
    uint64_t n = 0;
    memcpy(&n, sh->base, 8);
    if (n % 8) {
        err = path + ": header length " + std::to_string(n) + " is not a multiple of 8";
        return false;
    }
    sh->data0 = n + 8;
    if (n > sh->size - 8 || sh->data0 + 8 > sh->size) {  // n + 8 must not wrap
        err = path + ": header length exceeds the file";
        return false;
    }
    JVal root;
    JParser jp(reinterpret_cast<const char*>(sh->base + 8), n);
    if (!jp.parse(root) || root.kind != JVal::OBJ) {
        err = path + ": header is not a JSON object";
        return false;
    }
    hfmoe_safetensors_stats& s = ck.stats;
    std::set<std::string> seen;
    for (const auto& kv : root.obj) {
        const std::string& name = kv.first;
        if (name.empty() || name[0] == '_') continue;  // __metadata__
        ++s.total;
        auto reject = [&](uint64_t& why) {
            ++s.rejected;
            ++why;
        };
        const JVal& t = kv.second;
        if (t.kind != JVal::OBJ) {
            reject(s.shape_rejected);
            continue;
        }
        TensorRef ref;
        ref.shard = sh.get();
        const JVal* dt = t.get("dtype");
        if (dt && dt->kind == JVal::STR) ref.dtype = dt->str;
        const size_t eb = dtype_bytes(ref.dtype);
        if (!eb) {
            reject(s.dtype_rejected);
            continue;
        }
        if (ref.dtype != "BF16") {
            if (ref.dtype != "F32" || name.find("e_score_correction_bias") == std::string::npos) {
                reject(s.dtype_rejected);
                continue;
            }
            ++s.f32_allowed_accepted;
        }
        const JVal* shp = t.get("shape");
        bool ok = shp && shp->kind == JVal::ARR && !shp->arr.empty();
        uint64_t numel = 1;
        if (ok) {
            for (const JVal& dim : shp->arr) {
                if (dim.kind != JVal::NUM || dim.num < 0.0 || dim.num != std::floor(dim.num) ||
                    dim.num > (double)(1 << 30)) {
                    ok = false;
                    break;
                }
                const uint64_t dn = (uint64_t)dim.num;
                if (dn && numel > UINT64_MAX / dn) {  // the product must not wrap
                    ok = false;
                    break;
                }
                ref.shape.push_back((int64_t)dn);
                numel *= dn;
            }
        }
        if (!ok) {
            reject(s.shape_rejected);
            continue;
        }
        const JVal* off = t.get("data_offsets");
        // Offsets past the file are out of bounds; checking them as doubles
        // first keeps the integer conversion and data0 + end from wrapping.
        ok = off && off->kind == JVal::ARR && off->arr.size() == 2 && off->arr[0].kind == JVal::NUM &&
             off->arr[1].kind == JVal::NUM && off->arr[0].num >= 0.0 && off->arr[0].num <= off->arr[1].num &&
             off->arr[1].num <= (double)sh->size;
        if (ok) {
            ref.begin = (uint64_t)off->arr[0].num;
            ref.end = (uint64_t)off->arr[1].num;
            ok = ref.end > ref.begin;
        }
        if (!ok || sh->data0 + ref.end > sh->size) {
            reject(s.bounds_rejected);
            continue;
        }
        if ((sh->data0 + ref.begin) % 8) {
            reject(s.alignment_rejected);
            continue;
        }
        if (numel * eb != ref.bytes()) {
            reject(s.byte_mismatch_rejected);
            continue;
        }
        if (!seen.insert(name).second) {  // a second tensor of one name in this shard
            reject(s.duplicate_rejected);
            continue;
        }
        ++s.accepted;
        // With an index, a tensor is taken from the shard the index names for
        // it; without one, from the first shard (in file-name order) holding it.
        if (wanted) {
            auto w = wanted->find(name);
            if (w == wanted->end() || w->second != shard_name) continue;
        }
        ck.tensors.emplace(name, ref);
    }
    ++s.shards;
    ck.shards.push_back(std::move(sh));
    return true;
}

bool read_index(const std::string& path, std::map<std::string, std::string>& map, std::string& err) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) return false;
    std::string txt;
    char buf[1 << 16];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) txt.append(buf, n);
    fclose(f);
    JVal root;
    JParser jp(txt.data(), txt.size());
    const JVal* wm = nullptr;
    if (jp.parse(root) && root.kind == JVal::OBJ) wm = root.get("weight_map");
    if (!wm || wm->kind != JVal::OBJ) {
        err = path + ": no weight_map object";
        return false;
    }
    for (const auto& kv : wm->obj)
        if (kv.second.kind == JVal::STR) map.emplace(kv.first, kv.second.str);
    return true;
}

// Copies of one layer load.  Host-to-HBM copies go through a ring of pinned
// staging buffers: the host threads fill slot i (memcpy out of the mapped
// shard) while the copy stream moves slot i-1 to HBM; a slot is refilled
// only after its previous transfer finished.  Host-to-pinned copies are plain
// threaded memcpy.  The mapped pages are never handed to the runtime.
struct CopyJob {
    const uint8_t* src;
    void* dst;
    size_t bytes;
    bool to_device;
};

void parallel_memcpy(uint8_t* dst, const uint8_t* src, size_t bytes, int threads) {
    const size_t min_part = 4u << 20;
    const int n = (int)std::max<size_t>(1, std::min<size_t>((size_t)threads, bytes / min_part));
    if (n == 1) {
        memcpy(dst, src, bytes);
        return;
    }
    std::vector<std::thread> pool;
    const size_t part = (bytes + n - 1) / n;
    for (int i = 0; i < n; ++i) {
        const size_t b = (size_t)i * part, e = std::min(bytes, b + part);
        if (b < e) pool.emplace_back([=] { memcpy(dst + b, src + b, e - b); });
    }
    for (auto& t : pool) t.join();
}

hipError_t run_copies(const std::vector<CopyJob>& jobs) {
    const int threads = (int)std::min(16u, std::max(1u, std::thread::hardware_concurrency()));
    constexpr int kSlots = 4;
    constexpr size_t kSlotBytes = 32u << 20;
    uint8_t* stage[kSlots] = {};
    hipEvent_t done[kSlots] = {};
    bool busy[kSlots] = {};
    hipError_t e = hipSuccess;
    for (int i = 0; i < kSlots && e == hipSuccess; ++i) {
        e = hipHostMalloc(reinterpret_cast<void**>(&stage[i]), kSlotBytes, hipHostMallocDefault);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&done[i], hipEventDisableTiming);
    }
    int slot = 0;
    for (const CopyJob& j : jobs) {
        if (e != hipSuccess) break;
        if (!j.to_device) {
            parallel_memcpy(static_cast<uint8_t*>(j.dst), j.src, j.bytes, threads);
            continue;
        }
        for (size_t off = 0; off < j.bytes && e == hipSuccess; off += kSlotBytes) {
            const size_t n = std::min(kSlotBytes, j.bytes - off);
            if (busy[slot]) e = hipEventSynchronize(done[slot]);
            if (e != hipSuccess) break;
            parallel_memcpy(stage[slot], j.src + off, n, threads);
            e = hipMemcpyAsync(static_cast<uint8_t*>(j.dst) + off, stage[slot], n, hipMemcpyHostToDevice,
                               g.copy_stream);
            if (e == hipSuccess) e = hipEventRecord(done[slot], g.copy_stream);
            busy[slot] = true;
            slot = (slot + 1) % kSlots;
        }
    }
    const hipError_t s = hipStreamSynchronize(g.copy_stream);
    if (e == hipSuccess) e = s;
    for (int i = 0; i < kSlots; ++i) {
        if (done[i]) hipEventDestroy(done[i]);
        if (stage[i]) hipHostFree(stage[i]);
    }
    return e;
}

const TensorRef* find2(const hfmoe_checkpoint& ck, const std::string& name, int64_t r, int64_t c,
                       const char* dtype, std::string& err) {
    auto it = ck.tensors.find(name);
    if (it == ck.tensors.end()) {
        err = "tensor " + name + " is missing";
        return nullptr;
    }
    const TensorRef& t = it->second;
    const bool shape_ok = c > 0 ? (t.shape.size() == 2 && t.shape[0] == r && t.shape[1] == c)
                                : (t.shape.size() == 1 && t.shape[0] == r);
    if (!shape_ok || (dtype && t.dtype != dtype)) {
        std::string sh;
        for (size_t i = 0; i < t.shape.size(); ++i) sh += (i ? "," : "") + std::to_string(t.shape[i]);
        err = "tensor " + name + " is " + t.dtype + " [" + sh + "], expected " + (dtype ? dtype : "F32/BF16") +
              " [" + std::to_string(r) + (c > 0 ? "," + std::to_string(c) : "") + "]";
        return nullptr;
    }
    return &t;
}

}  // namespace
}  // namespace hf

using namespace hf;

extern "C" {

int hfmoe_checkpoint_open(const char* path, hfmoe_checkpoint** out) {
    if (!path || !out) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    auto ck = std::make_unique<hfmoe_checkpoint>();
    std::string err;
    struct stat st;
    if (stat(path, &st) != 0) return fail(HFMOE_ERR_INVALID_ARGUMENT, "%s does not exist", path);
    if (S_ISDIR(st.st_mode)) {
        const std::string dir(path);
        std::map<std::string, std::string> index;
        const bool have_index = read_index(dir + "/model.safetensors.index.json", index, err);
        if (!have_index && !err.empty()) return fail(HFMOE_ERR_INVALID_ARGUMENT, "%s", err.c_str());
        std::vector<std::string> files;
        if (DIR* d = opendir(path)) {
            while (dirent* e = readdir(d)) {
                const std::string f = e->d_name;
                if (ends_with(f, ".safetensors")) files.push_back(f);
            }
            closedir(d);
        }
        std::sort(files.begin(), files.end());
        if (files.empty()) return fail(HFMOE_ERR_INVALID_ARGUMENT, "no .safetensors files in %s", path);
        for (const std::string& f : files) {
            if (have_index) {
                bool used = false;
                for (const auto& kv : index) used |= kv.second == f;
                if (!used) continue;
            }
            if (!open_shard(*ck, dir + "/" + f, have_index ? &index : nullptr, f, err))
                return fail(HFMOE_ERR_INVALID_ARGUMENT, "%s", err.c_str());
        }
    } else {
        if (!open_shard(*ck, path, nullptr, "", err)) return fail(HFMOE_ERR_INVALID_ARGUMENT, "%s", err.c_str());
    }
    *out = ck.release();
    return HFMOE_OK;
}

int hfmoe_checkpoint_stats(const hfmoe_checkpoint* ck, hfmoe_safetensors_stats* out) {
    if (!ck || !out) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null argument");
    *out = ck->stats;
    return HFMOE_OK;
}

int hfmoe_checkpoint_tensor(const hfmoe_checkpoint* ck, const char* name, hfmoe_tensor_info* out) {
    if (!ck || !name || !out) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null argument");
    auto it = ck->tensors.find(name);
    if (it == ck->tensors.end()) return fail(HFMOE_ERR_NOT_REGISTERED, "tensor %s not in the checkpoint", name);
    const TensorRef& t = it->second;
    *out = hfmoe_tensor_info{};
    snprintf(out->dtype, sizeof out->dtype, "%s", t.dtype.c_str());
    out->ndim = (int32_t)std::min<size_t>(t.shape.size(), 8);
    for (int i = 0; i < out->ndim; ++i) out->shape[i] = t.shape[i];
    out->nbytes = t.bytes();
    out->file_offset = t.shard->data0 + t.begin;
    return HFMOE_OK;
}

int hfmoe_checkpoint_load_moe_layer(hfmoe_checkpoint* ck, int layer, int experts_location) {
    int rc = require_cfg();
    if (rc) return rc;
    if (!ck) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null checkpoint");
    if (experts_location != HFMOE_EXPERTS_DEVICE && experts_location != HFMOE_EXPERTS_HOST_PINNED)
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "unknown experts_location %d", experts_location);
    if (ck->loaded.count(layer)) return fail(HFMOE_ERR_INVALID_ARGUMENT, "layer %d already loaded", layer);
    const Cfg& c = g.cfg;
    const int64_t d = c.d, I = c.I, E = c.E, S = (int64_t)c.n_shared * c.I;
    const std::string pre = "model.layers." + std::to_string(layer) + ".mlp.";
    std::string err;
    const TensorRef* router = find2(*ck, pre + "gate.weight", E, d, "BF16", err);
    if (!router) return fail(HFMOE_ERR_INVALID_ARGUMENT, "%s", err.c_str());
    const TensorRef* bias = nullptr;
    if (ck->tensors.count(pre + "gate.e_score_correction_bias")) {
        bias = find2(*ck, pre + "gate.e_score_correction_bias", E, 0, nullptr, err);
        if (!bias) return fail(HFMOE_ERR_INVALID_ARGUMENT, "%s", err.c_str());
    }
    const TensorRef *sg = nullptr, *su = nullptr, *sd = nullptr;
    if (S > 0) {
        sg = find2(*ck, pre + "shared_experts.gate_proj.weight", S, d, "BF16", err);
        if (sg) su = find2(*ck, pre + "shared_experts.up_proj.weight", S, d, "BF16", err);
        if (su) sd = find2(*ck, pre + "shared_experts.down_proj.weight", d, S, "BF16", err);
        if (!sd) return fail(HFMOE_ERR_INVALID_ARGUMENT, "%s", err.c_str());
    }
    const TensorRef* norm = nullptr;
    const std::string norm_name = "model.layers." + std::to_string(layer) + ".post_attention_layernorm.weight";
    if (ck->tensors.count(norm_name)) {
        norm = find2(*ck, norm_name, d, 0, "BF16", err);
        if (!norm) return fail(HFMOE_ERR_INVALID_ARGUMENT, "%s", err.c_str());
    }
    std::vector<const TensorRef*> ex(3 * E);
    static const char* kProj[3] = {"gate_proj", "up_proj", "down_proj"};
    for (int64_t e = 0; e < E; ++e)
        for (int q = 0; q < 3; ++q) {
            const std::string nm = pre + "experts." + std::to_string(e) + "." + kProj[q] + ".weight";
            ex[3 * e + q] = find2(*ck, nm, q < 2 ? I : d, q < 2 ? d : I, "BF16", err);
            if (!ex[3 * e + q]) return fail(HFMOE_ERR_INVALID_ARGUMENT, "%s", err.c_str());
        }

    LoadedLayer L;
    auto cleanup = [&]() {
        for (void* p : L.dev) hipFree(p);
        for (void* p : L.host) hipHostFree(p);
    };
    std::vector<CopyJob> jobs;
    auto to_dev = [&](const void* src, size_t bytes, void** dst) -> hipError_t {
        hipError_t e = hipMalloc(dst, bytes);
        if (e != hipSuccess) return e;
        L.dev.push_back(*dst);
        jobs.push_back({static_cast<const uint8_t*>(src), *dst, bytes, true});
        return hipSuccess;
    };
    hipError_t e = hipSuccess;
    void *router_d = nullptr, *bias_d = nullptr, *sg_d = nullptr, *su_d = nullptr, *sd_d = nullptr, *norm_d = nullptr;
    e = to_dev(router->data(), router->bytes(), &router_d);
    std::vector<float> bias_f32;
    if (e == hipSuccess && bias) {
        bias_f32.resize(E);
        if (bias->dtype == "F32") {
            memcpy(bias_f32.data(), bias->data(), 4 * E);
        } else {  // BF16 bias: widened, as loadWeightToF32 does by dtype (glm_forward.cpp:171-183)
            const uint16_t* b = reinterpret_cast<const uint16_t*>(bias->data());
            for (int64_t i = 0; i < E; ++i) {
                const uint32_t u = (uint32_t)b[i] << 16;
                memcpy(&bias_f32[i], &u, 4);
            }
        }
        e = to_dev(bias_f32.data(), 4 * E, &bias_d);
    }
    if (e == hipSuccess && S > 0) e = to_dev(sg->data(), sg->bytes(), &sg_d);
    if (e == hipSuccess && S > 0) e = to_dev(su->data(), su->bytes(), &su_d);
    if (e == hipSuccess && S > 0) e = to_dev(sd->data(), sd->bytes(), &sd_d);
    if (e == hipSuccess && norm) e = to_dev(norm->data(), norm->bytes(), &norm_d);
    // Routed experts: one block, expert e at e * 3*I*d elements as [gate | up | down].
    const size_t proj = (size_t)I * d, eb = 3 * proj * 2;
    uint16_t* block = nullptr;
    const bool on_dev = experts_location == HFMOE_EXPERTS_DEVICE;
    if (e == hipSuccess) {
        if (on_dev) {
            e = hipMalloc(reinterpret_cast<void**>(&block), eb * E);
            if (e == hipSuccess) L.dev.push_back(block);
        } else {
            e = hipHostMalloc(reinterpret_cast<void**>(&block), eb * E, hipHostMallocDefault);
            if (e == hipSuccess) L.host.push_back(block);
        }
    }
    std::vector<const uint16_t*> table(3 * E);
    for (int64_t ei = 0; ei < E && e == hipSuccess; ++ei)
        for (int q = 0; q < 3; ++q) {
            uint16_t* dst = block + ei * 3 * proj + q * proj;
            table[3 * ei + q] = dst;
            jobs.push_back({ex[3 * ei + q]->data(), dst, proj * 2, on_dev});
        }
    if (e == hipSuccess) e = run_copies(jobs);
    if (e != hipSuccess) {
        cleanup();
        return fail_hip(e, "checkpoint layer upload");
    }
    hfmoe_layer_weights w{};
    w.router_dev = static_cast<const uint16_t*>(router_d);
    w.score_bias_dev = static_cast<const float*>(bias_d);
    w.shared_gate_dev = static_cast<const uint16_t*>(sg_d);
    w.shared_up_dev = static_cast<const uint16_t*>(su_d);
    w.shared_down_dev = static_cast<const uint16_t*>(sd_d);
    w.experts = table.data();
    w.post_attention_norm_dev = static_cast<const uint16_t*>(norm_d);
    w.experts_location = experts_location;
    rc = hfmoe_register_layer(layer, &w);
    if (rc) {
        cleanup();
        return rc;
    }
    ck->loaded[layer] = std::move(L);
    return HFMOE_OK;
}

int hfmoe_checkpoint_load_dense_layer(hfmoe_checkpoint* ck, int layer) {
    int rc = require_cfg();
    if (rc) return rc;
    if (!ck) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null checkpoint");
    if (ck->loaded.count(layer)) return fail(HFMOE_ERR_INVALID_ARGUMENT, "layer %d already loaded", layer);
    const int64_t d = g.cfg.d;
    const std::string pre = "model.layers." + std::to_string(layer) + ".";
    auto it = ck->tensors.find(pre + "mlp.gate_proj.weight");
    if (it == ck->tensors.end())
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "tensor %smlp.gate_proj.weight is missing", pre.c_str());
    const int64_t inter = it->second.shape.empty() ? 0 : it->second.shape[0];
    std::string err;
    const TensorRef* gt = find2(*ck, pre + "mlp.gate_proj.weight", inter, d, "BF16", err);
    const TensorRef* ut = gt ? find2(*ck, pre + "mlp.up_proj.weight", inter, d, "BF16", err) : nullptr;
    const TensorRef* dt = ut ? find2(*ck, pre + "mlp.down_proj.weight", d, inter, "BF16", err) : nullptr;
    if (!dt) return fail(HFMOE_ERR_INVALID_ARGUMENT, "%s", err.c_str());
    const TensorRef* norm = nullptr;
    if (ck->tensors.count(pre + "post_attention_layernorm.weight")) {
        norm = find2(*ck, pre + "post_attention_layernorm.weight", d, 0, "BF16", err);
        if (!norm) return fail(HFMOE_ERR_INVALID_ARGUMENT, "%s", err.c_str());
    }
    LoadedLayer L;
    std::vector<CopyJob> jobs;
    void* p[4] = {};
    const TensorRef* src[4] = {gt, ut, dt, norm};
    hipError_t e = hipSuccess;
    for (int i = 0; i < 4 && e == hipSuccess; ++i) {
        if (!src[i]) continue;
        e = hipMalloc(&p[i], src[i]->bytes());
        if (e == hipSuccess) {
            L.dev.push_back(p[i]);
            jobs.push_back({src[i]->data(), p[i], src[i]->bytes(), true});
        }
    }
    if (e == hipSuccess) e = run_copies(jobs);
    if (e != hipSuccess) {
        for (void* q : L.dev) hipFree(q);
        return fail_hip(e, "checkpoint dense layer upload");
    }
    hfmoe_dense_weights w{};
    w.gate_dev = static_cast<const uint16_t*>(p[0]);
    w.up_dev = static_cast<const uint16_t*>(p[1]);
    w.down_dev = static_cast<const uint16_t*>(p[2]);
    w.post_attention_norm_dev = static_cast<const uint16_t*>(p[3]);
    w.intermediate = (int32_t)inter;
    rc = hfmoe_register_dense_layer(layer, &w);
    if (rc) {
        for (void* q : L.dev) hipFree(q);
        return rc;
    }
    ck->loaded[layer] = std::move(L);
    return HFMOE_OK;
}

int hfmoe_checkpoint_load_lm_head(hfmoe_checkpoint* ck) {
    int rc = require_cfg();
    if (rc) return rc;
    if (!ck) return fail(HFMOE_ERR_INVALID_ARGUMENT, "null checkpoint");
    const int64_t d = g.cfg.d;
    auto it = ck->tensors.find("lm_head.weight");
    if (it == ck->tensors.end()) return fail(HFMOE_ERR_INVALID_ARGUMENT, "tensor lm_head.weight is missing");
    const int64_t vocab = it->second.shape.empty() ? 0 : it->second.shape[0];
    std::string err;
    const TensorRef* w = find2(*ck, "lm_head.weight", vocab, d, "BF16", err);
    const TensorRef* norm = nullptr;
    if (w && ck->tensors.count("model.norm.weight")) norm = find2(*ck, "model.norm.weight", d, 0, "BF16", err);
    if (!w || (ck->tensors.count("model.norm.weight") && !norm))
        return fail(HFMOE_ERR_INVALID_ARGUMENT, "%s", err.c_str());
    LoadedLayer L;
    std::vector<CopyJob> jobs;
    void* p[2] = {};
    const TensorRef* src[2] = {w, norm};
    hipError_t e = hipSuccess;
    for (int i = 0; i < 2 && e == hipSuccess; ++i) {
        if (!src[i]) continue;
        e = hipMalloc(&p[i], src[i]->bytes());
        if (e == hipSuccess) {
            L.dev.push_back(p[i]);
            jobs.push_back({src[i]->data(), p[i], src[i]->bytes(), true});
        }
    }
    if (e == hipSuccess) e = run_copies(jobs);
    if (e != hipSuccess) {
        for (void* q : L.dev) hipFree(q);
        return fail_hip(e, "checkpoint lm head upload");
    }
    rc = hfmoe_register_lm_head(static_cast<const uint16_t*>(p[0]), static_cast<const uint16_t*>(p[1]),
                                (int32_t)vocab);
    if (rc) {
        for (void* q : L.dev) hipFree(q);
        return rc;
    }
    for (void* q : ck->lm_head.dev) hipFree(q);
    ck->lm_head = std::move(L);
    return HFMOE_OK;
}

void hfmoe_checkpoint_close(hfmoe_checkpoint* ck) {
    if (!ck) return;
    for (auto& kv : ck->loaded) {
        // The layer's weights go with the checkpoint: unregister it first --
        // unless the layer id now holds another registration (after a
        // reconfigure or an explicit register call), which is left alone.
        auto it = g.layers.find(kv.first);
        const void* first = kv.second.dev.empty() ? nullptr : kv.second.dev[0];
        const bool ours = it != g.layers.end() && first &&
                          (it->second.dense ? it->second.dev.sg == first : it->second.dev.router == first);
        if (ours) {
            g.pool.policy.forget_layer(kv.first);
            if (g.stream) hipStreamSynchronize(g.stream);
            if (g.copy_stream) hipStreamSynchronize(g.copy_stream);
            if (it->second.etab_dev) hipFree(it->second.etab_dev);
            g.layers.erase(it);
        }
        for (void* p : kv.second.dev) hipFree(p);
        for (void* p : kv.second.host) hipHostFree(p);
    }
    if (!ck->lm_head.dev.empty()) {
        if (g.lm.w == ck->lm_head.dev[0]) {
            if (g.stream) hipStreamSynchronize(g.stream);
            lm_head_release();
        }
        for (void* p : ck->lm_head.dev) hipFree(p);
    }
    delete ck;
}

}  // extern "C"
