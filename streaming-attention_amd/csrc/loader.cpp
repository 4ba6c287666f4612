// Qwen3 checkpoints in safetensors format -> sa_qwen3 device weights.
//
// A safetensors file is an 8-byte little-endian header length N, N bytes of
// JSON (an object: tensor name -> {"dtype", "shape", "data_offsets": [begin,
// end]}, plus an optional "__metadata__" entry), then the tensor data, with
// offsets relative to the end of the header.  The reference reads a Qwen3
// checkpoint with load_qwen3_weights (tensor_cpp/src/qwen3_loader.cpp:188-296):
// every tensor read as BF16 and widened to fp32 host tensors, q/k/v
// concatenated into qkv_projs (:265-282), 28 layers and 16/8 heads of 128
// assumed (:217-221).  Here the header is parsed as JSON, the shapes are read
// from it and checked against each other, the dtype (BF16 or F32) and byte
// range of every tensor are verified, and the weights are uploaded into the
// device layouts of sa_qwen3_tensor_ptr (matrices bf16, norm weights fp32).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdint>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "safetensors.h"
#include "sa_internal.h"
#include "sa_qwen3.h"

namespace sa {
namespace {

using Entry = StEntry;

// Recursive-descent reader of the header JSON.  Strings support the JSON
// escapes (\uXXXX as UTF-8, surrogate pairs included); numbers other than
// the integers of "shape" and "data_offsets" are skipped unparsed.
class HeaderParser {
public:
    HeaderParser(const char* p, size_t n) : p_(p), e_(p + n) {}

    bool parse(std::map<std::string, Entry>& out) {
        if (!lit('{')) return bad("header is not a JSON object");
        if (lit('}')) return end();
        for (;;) {
            std::string key;
            if (!str(key) || !lit(':')) return bad("expected \"name\":");
            if (key == "__metadata__") {
                if (!skip_value()) return bad("malformed __metadata__");
            } else {
                if (out.count(key)) return bad("duplicate tensor " + key);
                if (!entry(out[key])) return bad(err_.empty() ? "malformed entry for " + key : err_);
            }
            if (lit(',')) continue;
            if (lit('}')) return end();
            return bad("expected ',' or '}'");
        }
    }
    const std::string& error() const { return err_; }

private:
    const char* p_;
    const char* e_;
    std::string err_;

    bool bad(const std::string& m) {
        if (err_.empty()) err_ = m;
        return false;
    }
    void ws() {
        while (p_ < e_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_;
    }
    bool lit(char c) {
        ws();
        if (p_ < e_ && *p_ == c) {
            ++p_;
            return true;
        }
        return false;
    }
    bool end() {
        ws();
        return p_ == e_ || bad("trailing bytes after the header object");
    }
    static void utf8(std::string& s, uint32_t cp) {
        if (cp < 0x80) {
            s += char(cp);
        } else if (cp < 0x800) {
            s += char(0xC0 | (cp >> 6));
            s += char(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            s += char(0xE0 | (cp >> 12));
            s += char(0x80 | ((cp >> 6) & 0x3F));
            s += char(0x80 | (cp & 0x3F));
        } else {
            s += char(0xF0 | (cp >> 18));
            s += char(0x80 | ((cp >> 12) & 0x3F));
            s += char(0x80 | ((cp >> 6) & 0x3F));
            s += char(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(uint32_t& v) {
        if (e_ - p_ < 4) return false;
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else return false;
        }
        return true;
    }
    bool str(std::string& s) {
        if (!lit('"')) return false;
        s.clear();
        while (p_ < e_) {
            const char c = *p_++;
            if (c == '"') return true;
            if (static_cast<unsigned char>(c) < 0x20) return false;
            if (c != '\\') {
                s += c;
                continue;
            }
            if (p_ >= e_) return false;
            const char x = *p_++;
            switch (x) {
                case '"': s += '"'; break;
                case '\\': s += '\\'; break;
                case '/': s += '/'; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'n': s += '\n'; break;
                case 'r': s += '\r'; break;
                case 't': s += '\t'; break;
                case 'u': {
                    uint32_t cp;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00) {
                        uint32_t lo;
                        if (e_ - p_ < 6 || p_[0] != '\\' || p_[1] != 'u') return false;
                        p_ += 2;
                        if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return false;
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    utf8(s, cp);
                    break;
                }
                default: return false;
            }
        }
        return false;
    }
    bool integer(int64_t& v) {
        ws();
        if (p_ >= e_ || *p_ < '0' || *p_ > '9') return false;
        uint64_t u = 0;
        while (p_ < e_ && *p_ >= '0' && *p_ <= '9') {
            const uint64_t d = *p_++ - '0';
            if (u > (uint64_t(INT64_MAX) - d) / 10) return false;
            u = u * 10 + d;
        }
        v = static_cast<int64_t>(u);
        return true;
    }
    bool int_array(std::vector<int64_t>& a) {
        if (!lit('[')) return false;
        a.clear();
        if (lit(']')) return true;
        for (;;) {
            int64_t v;
            if (!integer(v)) return false;
            a.push_back(v);
            if (lit(',')) continue;
            return lit(']');
        }
    }
    bool skip_value(int depth = 0) {
        ws();
        if (p_ >= e_ || depth > 64) return false;
        const char c = *p_;
        if (c == '"') {
            std::string s;
            return str(s);
        }
        if (c == '{' || c == '[') {
            const char close = c == '{' ? '}' : ']';
            ++p_;
            if (lit(close)) return true;
            for (;;) {
                if (c == '{') {
                    std::string k;
                    if (!str(k) || !lit(':')) return false;
                }
                if (!skip_value(depth + 1)) return false;
                if (lit(',')) continue;
                return lit(close);
            }
        }
        // number, true, false, null
        const char* s = p_;
        while (p_ < e_ && std::strchr(",}] \n\r\t", *p_) == nullptr) ++p_;
        return p_ > s;
    }
    bool entry(Entry& t) {
        if (!lit('{')) return false;
        bool has_dtype = false, has_shape = false, has_off = false;
        if (!lit('}')) {
            for (;;) {
                std::string f;
                if (!str(f) || !lit(':')) return false;
                if (f == "dtype") {
                    if (!str(t.dtype)) return false;
                    has_dtype = true;
                } else if (f == "shape") {
                    if (!int_array(t.shape)) return false;
                    has_shape = true;
                } else if (f == "data_offsets") {
                    std::vector<int64_t> o;
                    if (!int_array(o) || o.size() != 2 || o[1] < o[0]) return false;
                    t.begin = static_cast<uint64_t>(o[0]);
                    t.end = static_cast<uint64_t>(o[1]);
                    has_off = true;
                } else if (!skip_value()) {
                    return false;
                }
                if (lit(',')) continue;
                if (lit('}')) break;
                return false;
            }
        }
        return has_dtype && has_shape && has_off;
    }
};

}  // namespace

Checkpoint::~Checkpoint() {
    if (map_ != MAP_FAILED && map_ != nullptr) munmap(map_, size_);
    if (fd_ >= 0) close(fd_);
}

sa_status Checkpoint::open_file(const char* path) {
    if (!path) return fail(SA_EINVAL, "null path");
    fd_ = ::open(path, O_RDONLY);
    if (fd_ < 0) return fail(SA_EIO, std::string("cannot open ") + path + ": " + std::strerror(errno));
    struct stat st{};
    if (fstat(fd_, &st) != 0) return fail(SA_EIO, std::string("cannot stat ") + path);
    size_ = static_cast<size_t>(st.st_size);
    if (size_ < 8) return fail(SA_EIO, "file shorter than the 8-byte header length");
    map_ = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (map_ == MAP_FAILED) return fail(SA_EIO, std::string("cannot map ") + path);
    const unsigned char* b = static_cast<const unsigned char*>(map_);
    uint64_t n = 0;
    for (int i = 7; i >= 0; --i) n = (n << 8) | b[i];
    if (n > size_ - 8) return fail(SA_EIO, "header length past the end of the file");
    data_ = b + 8 + n;
    data_size_ = size_ - 8 - n;
    HeaderParser parser(reinterpret_cast<const char*>(b + 8), n);
    if (!parser.parse(tensors_)) return fail(SA_EIO, "safetensors header: " + parser.error());
    for (const auto& kv : tensors_) {
        const Entry& t = kv.second;
        const int es = elem_size(t.dtype);
        for (int64_t s : t.shape)
            if (s < 0) return fail(SA_EIO, kv.first + ": negative dimension");
        if (t.end > data_size_) return fail(SA_EIO, kv.first + ": data range past the end of the file");
        if (es > 0 && t.end - t.begin != static_cast<uint64_t>(t.numel()) * es)
            return fail(SA_EIO, kv.first + ": byte range does not match shape and dtype");
    }
    return SA_OK;
}

int Checkpoint::elem_size(const std::string& dtype) { return dtype == "BF16" ? 2 : dtype == "F32" ? 4 : 0; }

const StEntry* Checkpoint::find(const std::string& name) const {
    auto it = tensors_.find(name);
    return it == tensors_.end() ? nullptr : &it->second;
}

sa_status Checkpoint::need(const std::string& name, const std::vector<int64_t>& shape, const StEntry** out) const {
    const Entry* t = find(name);
    if (!t) return fail(SA_EINVAL, "tensor not found: " + name);
    if (elem_size(t->dtype) == 0) return fail(SA_EINVAL, name + ": dtype " + t->dtype + " not supported (BF16, F32)");
    if (t->shape != shape) {
        std::string got, want;
        for (int64_t s : t->shape) got += std::to_string(s) + ",";
        for (int64_t s : shape) want += std::to_string(s) + ",";
        return fail(SA_EINVAL, name + ": shape [" + got + "] where [" + want + "] was expected");
    }
    *out = t;
    return SA_OK;
}

void Checkpoint::to_f32(const StEntry& t, float* dst) const {
    const unsigned char* src = bytes(t);
    const size_t n = static_cast<size_t>(t.numel());
    if (t.dtype == "F32") {
        std::memcpy(dst, src, n * 4);
        return;
    }
    for (size_t i = 0; i < n; ++i) {   // bf16 is the top half of an fp32
        uint16_t b;
        std::memcpy(&b, src + 2 * i, 2);
        const uint32_t u = static_cast<uint32_t>(b) << 16;
        std::memcpy(dst + i, &u, 4);
    }
}

int Checkpoint::num_layers() const {
    int n = 0;
    const std::string pre = "model.layers.";
    for (const auto& kv : tensors_) {
        const std::string& k = kv.first;
        if (k.compare(0, pre.size(), pre) != 0) continue;
        size_t i = pre.size();
        long v = 0;
        bool digits = false;
        while (i < k.size() && k[i] >= '0' && k[i] <= '9' && v < 1000000) {
            v = v * 10 + (k[i++] - '0');
            digits = true;
        }
        if (digits && i < k.size() && k[i] == '.') n = std::max<long>(n, v + 1);
    }
    return n;
}

std::string layer_tensor_name(int i, const char* leaf) { return "model.layers." + std::to_string(i) + "." + leaf; }

sa_status read_qwen3_desc(const Checkpoint& ck, sa_qwen3_desc* d) {
    const Entry* embed = ck.find("model.embed_tokens.weight");
    if (!embed) return fail(SA_EINVAL, "tensor not found: model.embed_tokens.weight");
    if (embed->shape.size() != 2) return fail(SA_EINVAL, "model.embed_tokens.weight must be 2-D");
    const int n_layers = ck.num_layers();
    if (n_layers <= 0) return fail(SA_EINVAL, "no model.layers.* tensors");
    const Entry* qn = ck.find(layer_tensor_name(0, "self_attn.q_norm.weight"));
    const Entry* qp = ck.find(layer_tensor_name(0, "self_attn.q_proj.weight"));
    const Entry* kp = ck.find(layer_tensor_name(0, "self_attn.k_proj.weight"));
    const Entry* gp = ck.find(layer_tensor_name(0, "mlp.gate_proj.weight"));
    if (!qn || !qp || !kp || !gp) return fail(SA_EINVAL, "layer 0 lacks q_norm, q_proj, k_proj or gate_proj");
    if (qn->shape.size() != 1 || qp->shape.size() != 2 || kp->shape.size() != 2 || gp->shape.size() != 2)
        return fail(SA_EINVAL, "layer 0 tensors have unexpected ranks");
    const int64_t D = qn->shape[0];
    if (D <= 0 || qp->shape[0] % D || kp->shape[0] % D)
        return fail(SA_EINVAL, "q_proj / k_proj rows are not multiples of head_dim");
    sa_qwen3_desc r{};
    r.num_layers = n_layers;
    r.vocab = static_cast<int>(embed->shape[0]);
    r.hidden = static_cast<int>(embed->shape[1]);
    r.head_dim = static_cast<int>(D);
    r.n_q_heads = static_cast<int>(qp->shape[0] / D);
    r.n_kv_heads = static_cast<int>(kp->shape[0] / D);
    r.intermediate = static_cast<int>(gp->shape[0]);
    r.max_pos = 0;
    r.rms_eps = 1e-6f;
    r.rope_theta = 1e6f;
    *d = r;
    return SA_OK;
}

namespace {

uint16_t f32_to_bf16_rne(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((u >> 16) | 0x0040u);   // quiet NaN
    u += 0x7FFFu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// Copy tensor t into the device tensor (layer, which) at element offset off.
sa_status upload(sa_qwen3* model, int layer, sa_qwen3_tensor which, size_t off, const Checkpoint& ck,
                 const Entry& t, const std::string& name) {
    void* ptr = nullptr;
    size_t count = 0;
    sa_dtype dt;
    sa_status s = sa_qwen3_tensor_ptr(model, layer, which, &ptr, &count, &dt);
    if (s != SA_OK) return s;
    const size_t n = static_cast<size_t>(t.numel());
    if (off + n > count) return fail(SA_EINVAL, name + ": does not fit the model tensor");
    const unsigned char* src = ck.bytes(t);
    if (dt == SA_DTYPE_BF16) {
        uint16_t* dst = static_cast<uint16_t*>(ptr) + off;
        if (t.dtype == "BF16") {
            SA_HIP_TRY(hipMemcpy(dst, src, n * 2, hipMemcpyHostToDevice));
        } else {
            std::vector<uint16_t> h(n);
            for (size_t i = 0; i < n; ++i) {
                float f;
                std::memcpy(&f, src + 4 * i, 4);
                h[i] = f32_to_bf16_rne(f);
            }
            SA_HIP_TRY(hipMemcpy(dst, h.data(), n * 2, hipMemcpyHostToDevice));
        }
    } else {
        float* dst = static_cast<float*>(ptr) + off;
        if (t.dtype == "F32") {
            SA_HIP_TRY(hipMemcpy(dst, src, n * 4, hipMemcpyHostToDevice));
        } else {
            std::vector<float> h(n);
            ck.to_f32(t, h.data());
            SA_HIP_TRY(hipMemcpy(dst, h.data(), n * 4, hipMemcpyHostToDevice));
        }
    }
    return SA_OK;
}

}  // namespace
}  // namespace sa

using namespace sa;

extern "C" sa_status sa_qwen3_desc_from_safetensors(const char* path, sa_qwen3_desc* desc) {
    clear_error();
    if (!desc) return fail(SA_EINVAL, "null desc");
    Checkpoint ck;
    sa_status s = ck.open_file(path);
    if (s != SA_OK) return s;
    return read_qwen3_desc(ck, desc);
}

extern "C" sa_status sa_qwen3_load_safetensors(sa_qwen3* model, const char* path) {
    clear_error();
    if (!model) return fail(SA_EINVAL, "null model");
    sa_qwen3_desc md{};
    sa_status s = sa_qwen3_get_desc(model, &md);
    if (s != SA_OK) return s;
    Checkpoint ck;
    if ((s = ck.open_file(path)) != SA_OK) return s;
    sa_qwen3_desc fd{};
    if ((s = read_qwen3_desc(ck, &fd)) != SA_OK) return s;
    if (fd.num_layers != md.num_layers || fd.hidden != md.hidden || fd.intermediate != md.intermediate ||
        fd.vocab != md.vocab || fd.n_q_heads != md.n_q_heads || fd.n_kv_heads != md.n_kv_heads ||
        fd.head_dim != md.head_dim)
        return fail(SA_EINVAL, "checkpoint shape (layers " + std::to_string(fd.num_layers) + ", hidden " +
                                   std::to_string(fd.hidden) + ", intermediate " + std::to_string(fd.intermediate) +
                                   ", vocab " + std::to_string(fd.vocab) + ", heads " +
                                   std::to_string(fd.n_q_heads) + "/" + std::to_string(fd.n_kv_heads) + " x " +
                                   std::to_string(fd.head_dim) + ") does not match the model");
    const int64_t H = md.hidden, I = md.intermediate, V = md.vocab, D = md.head_dim;
    const int64_t Nq = md.n_q_heads * D, Nk = md.n_kv_heads * D;
    const Entry* t = nullptr;
    auto put = [&](int layer, sa_qwen3_tensor which, size_t off, const std::string& name,
                   std::vector<int64_t> shape) -> sa_status {
        sa_status r = ck.need(name, std::move(shape), &t);
        if (r != SA_OK) return r;
        return upload(model, layer, which, off, ck, *t, name);
    };
    if ((s = put(0, SA_QW_EMBED, 0, "model.embed_tokens.weight", {V, H})) != SA_OK) return s;
    if ((s = put(0, SA_QW_FINAL_NORM, 0, "model.norm.weight", {H})) != SA_OK) return s;
    if (ck.find("lm_head.weight")) {
        if ((s = put(0, SA_QW_LM_HEAD, 0, "lm_head.weight", {V, H})) != SA_OK) return s;
    } else {   // tied word embeddings
        if ((s = put(0, SA_QW_LM_HEAD, 0, "model.embed_tokens.weight", {V, H})) != SA_OK) return s;
    }
    for (int l = 0; l < md.num_layers; ++l) {
        if ((s = put(l, SA_QW_IN_NORM, 0, layer_tensor_name(l, "input_layernorm.weight"), {H})) != SA_OK ||
            (s = put(l, SA_QW_POST_NORM, 0, layer_tensor_name(l, "post_attention_layernorm.weight"), {H})) != SA_OK ||
            (s = put(l, SA_QW_QKV, 0, layer_tensor_name(l, "self_attn.q_proj.weight"), {Nq, H})) != SA_OK ||
            (s = put(l, SA_QW_QKV, Nq * H, layer_tensor_name(l, "self_attn.k_proj.weight"), {Nk, H})) != SA_OK ||
            (s = put(l, SA_QW_QKV, (Nq + Nk) * H, layer_tensor_name(l, "self_attn.v_proj.weight"), {Nk, H})) != SA_OK ||
            (s = put(l, SA_QW_Q_NORM, 0, layer_tensor_name(l, "self_attn.q_norm.weight"), {D})) != SA_OK ||
            (s = put(l, SA_QW_K_NORM, 0, layer_tensor_name(l, "self_attn.k_norm.weight"), {D})) != SA_OK ||
            (s = put(l, SA_QW_O, 0, layer_tensor_name(l, "self_attn.o_proj.weight"), {H, Nq})) != SA_OK ||
            (s = put(l, SA_QW_GATE_UP, 0, layer_tensor_name(l, "mlp.gate_proj.weight"), {I, H})) != SA_OK ||
            (s = put(l, SA_QW_GATE_UP, I * H, layer_tensor_name(l, "mlp.up_proj.weight"), {I, H})) != SA_OK ||
            (s = put(l, SA_QW_DOWN, 0, layer_tensor_name(l, "mlp.down_proj.weight"), {H, I})) != SA_OK)
            return s;
    }
    return SA_OK;
}
