// checkpoint.cpp — safetensors reading / writing, quantized-weight loading
// and the offline quantizer (declarations and reference map in
// checkpoint.h), plus the C ABI of include/qimg_ckpt.h.
#include "checkpoint.h"

#include <cctype>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>

#include "qimg_ckpt.h"

namespace {

// ---- a JSON reader for safetensors headers and index files ---------------
struct Json {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0.0;
    int64_t inum = 0;
    bool is_int = false;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;  // document order

    const Json* get(const std::string& k) const {
        for (auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

class JsonReader {
public:
    explicit JsonReader(const std::string& s) : s_(s) {}
    bool parse(Json& out, std::string& err) {
        if (!value(out, 0) || (ws(), p_ != s_.size())) {
            err = "malformed JSON at byte " + std::to_string(p_);
            return false;
        }
        return true;
    }

private:
    const std::string& s_;
    size_t p_ = 0;
    void ws() {
        while (p_ < s_.size() && (s_[p_] == ' ' || s_[p_] == '\t' || s_[p_] == '\n' || s_[p_] == '\r')) ++p_;
    }
    bool lit(const char* w) {
        const size_t n = strlen(w);
        if (s_.compare(p_, n, w) != 0) return false;
        p_ += n;
        return true;
    }
    static void utf8(std::string& o, uint32_t c) {
        if (c < 0x80) {
            o += static_cast<char>(c);
        } else if (c < 0x800) {
            o += static_cast<char>(0xC0 | (c >> 6));
            o += static_cast<char>(0x80 | (c & 0x3F));
        } else if (c < 0x10000) {
            o += static_cast<char>(0xE0 | (c >> 12));
            o += static_cast<char>(0x80 | ((c >> 6) & 0x3F));
            o += static_cast<char>(0x80 | (c & 0x3F));
        } else {
            o += static_cast<char>(0xF0 | (c >> 18));
            o += static_cast<char>(0x80 | ((c >> 12) & 0x3F));
            o += static_cast<char>(0x80 | ((c >> 6) & 0x3F));
            o += static_cast<char>(0x80 | (c & 0x3F));
        }
    }
    bool hex4(uint32_t& c) {
        if (p_ + 4 > s_.size()) return false;
        c = 0;
        for (int i = 0; i < 4; ++i) {
            const char h = s_[p_++];
            c <<= 4;
            if (h >= '0' && h <= '9') c |= h - '0';
            else if (h >= 'a' && h <= 'f') c |= h - 'a' + 10;
            else if (h >= 'A' && h <= 'F') c |= h - 'A' + 10;
            else return false;
        }
        return true;
    }
    bool string(std::string& o) {
        if (p_ >= s_.size() || s_[p_] != '"') return false;
        ++p_;
        while (p_ < s_.size()) {
            const char c = s_[p_++];
            if (c == '"') return true;
            if (c != '\\') {
                o += c;
                continue;
            }
            if (p_ >= s_.size()) return false;
            const char e = s_[p_++];
            switch (e) {
                case '"': o += '"'; break;
                case '\\': o += '\\'; break;
                case '/': o += '/'; break;
                case 'b': o += '\b'; break;
                case 'f': o += '\f'; break;
                case 'n': o += '\n'; break;
                case 'r': o += '\r'; break;
                case 't': o += '\t'; break;
                case 'u': {
                    uint32_t c1;
                    if (!hex4(c1)) return false;
                    if (c1 >= 0xD800 && c1 < 0xDC00 && s_.compare(p_, 2, "\\u") == 0) {
                        p_ += 2;
                        uint32_t c2;
                        if (!hex4(c2) || c2 < 0xDC00 || c2 >= 0xE000) return false;
                        c1 = 0x10000 + ((c1 - 0xD800) << 10) + (c2 - 0xDC00);
                    }
                    utf8(o, c1);
                    break;
                }
                default: return false;
            }
        }
        return false;
    }
    bool value(Json& v, int depth) {
        if (depth > 64) return false;
        ws();
        if (p_ >= s_.size()) return false;
        const char c = s_[p_];
        if (c == '{') {
            v.kind = Json::Obj;
            ++p_;
            ws();
            if (p_ < s_.size() && s_[p_] == '}') return ++p_, true;
            for (;;) {
                ws();
                std::string k;
                if (!string(k)) return false;
                ws();
                if (p_ >= s_.size() || s_[p_++] != ':') return false;
                Json x;
                if (!value(x, depth + 1)) return false;
                v.obj.emplace_back(std::move(k), std::move(x));
                ws();
                if (p_ < s_.size() && s_[p_] == ',') { ++p_; continue; }
                if (p_ < s_.size() && s_[p_] == '}') return ++p_, true;
                return false;
            }
        }
        if (c == '[') {
            v.kind = Json::Arr;
            ++p_;
            ws();
            if (p_ < s_.size() && s_[p_] == ']') return ++p_, true;
            for (;;) {
                Json x;
                if (!value(x, depth + 1)) return false;
                v.arr.push_back(std::move(x));
                ws();
                if (p_ < s_.size() && s_[p_] == ',') { ++p_; continue; }
                if (p_ < s_.size() && s_[p_] == ']') return ++p_, true;
                return false;
            }
        }
        if (c == '"') return v.kind = Json::Str, string(v.str);
        if (lit("true")) return v.kind = Json::Bool, v.b = true, true;
        if (lit("false")) return v.kind = Json::Bool, true;
        if (lit("null")) return v.kind = Json::Null, true;
        const size_t b = p_;
        if (p_ < s_.size() && s_[p_] == '-') ++p_;
        bool frac = false;
        while (p_ < s_.size() && (isdigit(static_cast<unsigned char>(s_[p_])) || s_[p_] == '.' || s_[p_] == 'e' ||
                                  s_[p_] == 'E' || s_[p_] == '+' || s_[p_] == '-')) {
            frac |= !isdigit(static_cast<unsigned char>(s_[p_]));
            ++p_;
        }
        if (p_ == b) return false;
        const std::string t = s_.substr(b, p_ - b);
        v.kind = Json::Num;
        v.num = strtod(t.c_str(), nullptr);
        if (!frac && !(t.size() == 1 && t[0] == '-')) {
            v.is_int = true;
            v.inum = strtoll(t.c_str(), nullptr, 10);
        }
        return true;
    }
};

// safetensors.h:79-97, with F8_E4M3 added
bool parse_dtype(const std::string& s, DType& dt) {
    if (s == "BF16" || s == "bfloat16") dt = DType::BF16;
    else if (s == "F32" || s == "float32") dt = DType::FP32;
    else if (s == "F16" || s == "float16") dt = DType::FP16;
    else if (s == "I8" || s == "int8") dt = DType::INT8;
    else if (s == "U8" || s == "uint8") dt = DType::UINT8;
    else if (s == "I32" || s == "int32") dt = DType::INT32;
    else if (s == "F8_E4M3") dt = DType::FP8_E4M3;
    else return false;
    return true;
}

std::string escape_json(const std::string& s) {  // safetensors_writer.h:94-102
    std::string o;
    for (char c : s) {
        if (c == '"') o += "\\\"";
        else if (c == '\\') o += "\\\\";
        else o += c;
    }
    return o;
}

bool file_exists(const std::string& p) {
    std::ifstream f(p);
    return f.good();
}

}  // namespace

// ---- SafeTensorsWriter -----------------------------------------------------
void SafeTensorsWriter::add(const std::string& name, const std::string& dtype_str, const std::vector<int64_t>& shape,
                            const void* data_ptr, size_t nbytes) {
    Entry e;
    e.name = name;
    e.dtype_str = dtype_str;
    e.shape = shape;
    e.data.resize(nbytes);
    if (nbytes) memcpy(e.data.data(), data_ptr, nbytes);
    entries_.push_back(std::move(e));
}

bool SafeTensorsWriter::write(const std::string& filepath) const {
    std::string h = "{";
    size_t off = 0;
    for (size_t i = 0; i < entries_.size(); ++i) {
        const Entry& e = entries_[i];
        if (i) h += ",";
        h += "\"" + escape_json(e.name) + "\":{\"dtype\":\"" + e.dtype_str + "\",\"shape\":[";
        for (size_t j = 0; j < e.shape.size(); ++j) h += (j ? "," : "") + std::to_string(e.shape[j]);
        h += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + e.data.size()) + "]}";
        off += e.data.size();
    }
    h += "}";
    while ((8 + h.size()) % 8 != 0) h += ' ';
    FILE* f = fopen(filepath.c_str(), "wb");
    if (!f) {
        fprintf(stderr, "SafeTensorsWriter: failed to open %s for writing\n", filepath.c_str());
        return false;
    }
    uint8_t len[8];
    const uint64_t n = h.size();
    for (int i = 0; i < 8; ++i) len[i] = static_cast<uint8_t>(n >> (8 * i));  // little endian
    bool ok = fwrite(len, 1, 8, f) == 8 && fwrite(h.data(), 1, h.size(), f) == h.size();
    for (const Entry& e : entries_)
        ok = ok && fwrite(e.data.data(), 1, e.data.size(), f) == e.data.size();
    ok = (fclose(f) == 0) && ok;
    if (!ok) fprintf(stderr, "SafeTensorsWriter: failed writing %s\n", filepath.c_str());
    return ok;
}

// ---- SafeTensorsLoader -----------------------------------------------------
bool SafeTensorsLoader::load_file(const std::string& filepath) {
    FILE* f = fopen(filepath.c_str(), "rb");
    if (!f) return error_ = "failed to open " + filepath, false;
    uint8_t len[8];
    std::string header;
    bool ok = fread(len, 1, 8, f) == 8;
    uint64_t n = 0;
    for (int i = 0; i < 8; ++i) n |= static_cast<uint64_t>(len[i]) << (8 * i);
    fseek(f, 0, SEEK_END);
    const long fsize = ftell(f);
    ok = ok && fsize >= 8 && n <= static_cast<uint64_t>(fsize - 8) && n < (1ull << 30);
    if (ok) {
        header.resize(n);
        fseek(f, 8, SEEK_SET);
        ok = fread(&header[0], 1, n, f) == n;
    }
    fclose(f);
    if (!ok) return error_ = filepath + ": truncated or invalid safetensors header", false;
    Json root;
    std::string err;
    if (!JsonReader(header).parse(root, err) || root.kind != Json::Obj)
        return error_ = filepath + ": " + (err.empty() ? "header is not an object" : err), false;
    const size_t data_len = static_cast<size_t>(fsize) - 8 - n;
    std::vector<TensorInfo> add;
    for (auto& kv : root.obj) {
        if (kv.first == "__metadata__") continue;
        const Json& v = kv.second;
        const Json* dt = v.get("dtype");
        const Json* sh = v.get("shape");
        const Json* of = v.get("data_offsets");
        if (!dt || dt->kind != Json::Str || !sh || sh->kind != Json::Arr || !of || of->kind != Json::Arr ||
            of->arr.size() != 2 || !of->arr[0].is_int || !of->arr[1].is_int)
            return error_ = filepath + ": malformed entry for tensor '" + kv.first + "'", false;
        TensorInfo t;
        t.name = kv.first;
        t.filename = filepath;
        t.dtype_str = dt->str;
        if (!parse_dtype(dt->str, t.dtype))
            return error_ = filepath + ": unknown dtype '" + dt->str + "' for tensor '" + kv.first + "'", false;
        int64_t numel = 1;
        for (auto& d : sh->arr) {
            if (!d.is_int || d.inum < 0) return error_ = filepath + ": bad shape for '" + kv.first + "'", false;
            t.shape.push_back(d.inum);
            numel *= d.inum;
        }
        const int64_t b = of->arr[0].inum, e = of->arr[1].inum;
        if (b < 0 || e < b || static_cast<size_t>(e) > data_len ||
            static_cast<size_t>(e - b) != static_cast<size_t>(numel) * dtype_size(t.dtype))
            return error_ = filepath + ": data_offsets of '" + kv.first + "' do not match its shape and dtype", false;
        t.data_offset = static_cast<size_t>(b);
        t.nbytes = static_cast<size_t>(e - b);
        add.push_back(std::move(t));
    }
    files_.push_back({filepath, 8 + static_cast<size_t>(n)});
    for (auto& t : add) {
        if (!find(t.name)) order_.push_back(t.name);
        tensors_.push_back(std::move(t));
    }
    return true;
}

bool SafeTensorsLoader::load_sharded(const std::string& index_path) {
    std::ifstream ifs(index_path);
    if (!ifs.good()) return error_ = "failed to open index " + index_path, false;
    const std::string content((std::istreambuf_iterator<char>(ifs)), std::istreambuf_iterator<char>());
    Json root;
    std::string err;
    if (!JsonReader(content).parse(root, err)) return error_ = index_path + ": " + err, false;
    const Json* wm = root.get("weight_map");
    if (!wm || wm->kind != Json::Obj) return error_ = index_path + ": no weight_map", false;
    const size_t slash = index_path.find_last_of('/');
    const std::string dir = slash == std::string::npos ? "" : index_path.substr(0, slash + 1);
    std::vector<std::string> shards;
    for (auto& kv : wm->obj) {
        if (kv.second.kind != Json::Str) return error_ = index_path + ": bad weight_map entry", false;
        bool seen = false;
        for (auto& s : shards) seen |= (s == kv.second.str);
        if (!seen) shards.push_back(kv.second.str);
    }
    for (auto& s : shards)
        if (!load_file(dir + s)) return false;
    return true;
}

const TensorInfo* SafeTensorsLoader::find(const std::string& name) const {
    // the last file that holds a name wins, as the reference's map assignment
    for (size_t i = tensors_.size(); i-- > 0;)
        if (tensors_[i].name == name) return &tensors_[i];
    return nullptr;
}

bool SafeTensorsLoader::has_tensor(const std::string& name) const { return find(name) != nullptr; }

const TensorInfo& SafeTensorsLoader::get_info(const std::string& name) const {
    const TensorInfo* t = find(name);
    if (!t) {
        fprintf(stderr, "Tensor not found: %s\n", name.c_str());
        exit(1);
    }
    return *t;
}

size_t SafeTensorsLoader::data_start(const std::string& filename) const {
    for (auto& f : files_)
        if (f.filepath == filename) return f.data_start;
    return 0;
}

std::vector<uint8_t> SafeTensorsLoader::read_bytes(const std::string& name) const {
    const TensorInfo& t = get_info(name);
    std::vector<uint8_t> buf(t.nbytes);
    FILE* f = fopen(t.filename.c_str(), "rb");
    if (!f) {
        fprintf(stderr, "Failed to open: %s\n", t.filename.c_str());
        exit(1);
    }
    const bool ok = fseek(f, static_cast<long>(data_start(t.filename) + t.data_offset), SEEK_SET) == 0 &&
                    fread(buf.data(), 1, t.nbytes, f) == t.nbytes;
    fclose(f);
    if (!ok) {
        fprintf(stderr, "Failed to read tensor: %s\n", name.c_str());
        exit(1);
    }
    return buf;
}

Tensor SafeTensorsLoader::load_tensor(const std::string& name) const {
    const TensorInfo& t = get_info(name);
    const std::vector<uint8_t> buf = read_bytes(name);
    Tensor d = Tensor::alloc(t.shape, t.dtype);
    if (!buf.empty()) d.from_host(buf.data(), buf.size());
    return d;
}

bool load_model_dir(const std::string& dir, SafeTensorsLoader& loader) {
    if (dir.size() > 12 && dir.compare(dir.size() - 12, 12, ".safetensors") == 0) return loader.load_file(dir);
    for (const char* n : {"/model.safetensors", "/diffusion_pytorch_model.safetensors"})
        if (file_exists(dir + n)) return loader.load_file(dir + n);
    for (const char* n : {"/model.safetensors.index.json", "/diffusion_pytorch_model.safetensors.index.json"})
        if (file_exists(dir + n)) return loader.load_sharded(dir + n);
    fprintf(stderr, "No safetensors files found in %s\n", dir.c_str());
    return false;
}

// ---- quantized weights -------------------------------------------------------
CheckpointKind detect_checkpoint(const SafeTensorsLoader& loader) {
    // a block-level weight, not the boundary layers (kept BF16)
    const std::string probe = "transformer_blocks.0.attn.to_q.weight";
    if (loader.has_tensor(probe)) {
        const DType dt = loader.get_info(probe).dtype;
        if (dt == DType::INT8) return CheckpointKind::INT8;
        if (dt == DType::FP8_E4M3) return CheckpointKind::FP8;
    }
    return CheckpointKind::BF16;
}

QuantizedWeight load_quantized_weight(const SafeTensorsLoader& loader, const std::string& name, bool keep_bf16) {
    const TensorInfo& info = loader.get_info(name);
    if (info.dtype == DType::INT8 || info.dtype == DType::FP8_E4M3) {
        if (info.shape.size() != 2 || !loader.has_tensor(name + ".__scales__")) {
            fprintf(stderr, "load_quantized_weight: %s needs a 2-D shape and %s.__scales__\n", name.c_str(),
                    name.c_str());
            exit(1);
        }
        const TensorInfo& si = loader.get_info(name + ".__scales__");
        if (si.dtype != DType::FP32 || si.shape.size() != 1 || si.shape[0] != info.shape[0]) {
            fprintf(stderr, "load_quantized_weight: %s.__scales__ must be F32 [%lld]\n", name.c_str(),
                    static_cast<long long>(info.shape[0]));
            exit(1);
        }
        QuantizedWeight qw;
        qw.mode = info.dtype == DType::INT8 ? QuantMode::INT8_HADAMARD : QuantMode::FP8_HADAMARD;
        qw.data = loader.load_tensor(name);
        qw.scales = loader.load_tensor(name + ".__scales__");
        qw.had_block_size = hadamard_block_size(static_cast<int>(info.shape[1]));
        return qw;
    }
    if (info.dtype == DType::BF16 && keep_bf16) {
        QuantizedWeight qw;
        qw.mode = QuantMode::BF16;
        qw.data = loader.load_tensor(name);
        return qw;
    }
    Tensor bf16 = loader.load_tensor(name);
    QuantizedWeight qw = quantize_weight_tensor(bf16);
    bf16.free_data();
    return qw;
}

std::vector<std::pair<std::string, bool>> quantize_plan(int num_blocks) {
    std::vector<std::pair<std::string, bool>> p;
    auto q = [&](const std::string& n) { p.emplace_back(n, true); };
    auto c = [&](const std::string& n) { p.emplace_back(n, false); };
    q("time_text_embed.timestep_embedder.linear_1.weight");
    c("time_text_embed.timestep_embedder.linear_1.bias");
    q("time_text_embed.timestep_embedder.linear_2.weight");
    c("time_text_embed.timestep_embedder.linear_2.bias");
    for (const char* n : {"txt_norm.weight", "img_in.weight", "img_in.bias", "txt_in.weight", "txt_in.bias",
                          "norm_out.linear.weight", "norm_out.linear.bias", "proj_out.weight", "proj_out.bias"})
        c(n);
    for (int i = 0; i < num_blocks; ++i) {
        const std::string b = "transformer_blocks." + std::to_string(i) + ".";
        q(b + "img_mod.1.weight");
        c(b + "img_mod.1.bias");
        q(b + "txt_mod.1.weight");
        c(b + "txt_mod.1.bias");
        for (const char* s : {"q", "k", "v"}) q(b + "attn.to_" + s + ".weight");
        for (const char* s : {"q", "k", "v"}) c(b + "attn.to_" + s + ".bias");
        c(b + "attn.norm_q.weight");
        c(b + "attn.norm_k.weight");
        for (const char* s : {"q", "k", "v"}) q(b + "attn.add_" + s + "_proj.weight");
        for (const char* s : {"q", "k", "v"}) c(b + "attn.add_" + s + "_proj.bias");
        c(b + "attn.norm_added_q.weight");
        c(b + "attn.norm_added_k.weight");
        q(b + "attn.to_out.0.weight");
        c(b + "attn.to_out.0.bias");
        q(b + "attn.to_add_out.weight");
        c(b + "attn.to_add_out.bias");
        for (const char* m : {"img_mlp", "txt_mlp"}) {
            q(b + m + ".net.0.proj.weight");
            c(b + m + ".net.0.proj.bias");
            q(b + m + ".net.2.weight");
            c(b + m + ".net.2.bias");
        }
    }
    return p;
}

bool quantize_checkpoint(const std::string& in, const std::string& out, QuantMode mode, int num_blocks,
                         std::string* err) {
    auto fail = [&](const std::string& m) {
        if (err) *err = m;
        return false;
    };
    if (mode != QuantMode::INT8_HADAMARD && mode != QuantMode::FP8_HADAMARD)
        return fail("quantize_checkpoint: mode must be INT8_HADAMARD or FP8_HADAMARD");
    if (num_blocks < 0) return fail("quantize_checkpoint: num_blocks must be >= 0");
    SafeTensorsLoader loader;
    if (!load_model_dir(in, loader))
        return fail(loader.error().empty() ? "no safetensors checkpoint at " + in : loader.error());
    const auto plan = quantize_plan(num_blocks);
    for (auto& e : plan)
        if (!loader.has_tensor(e.first)) return fail("tensor not found in checkpoint: " + e.first);
    SafeTensorsWriter writer;
    const char* qdt = mode == QuantMode::INT8_HADAMARD ? "I8" : "F8_E4M3";
    for (auto& e : plan) {
        const TensorInfo& info = loader.get_info(e.first);
        if (!e.second) {  // quantize.cu:139-161: raw bytes, F32 kept, anything else labelled BF16
            const std::vector<uint8_t> buf = loader.read_bytes(e.first);
            writer.add(e.first, info.dtype == DType::FP32 ? "F32" : "BF16", info.shape, buf.data(), buf.size());
            continue;
        }
        if (info.dtype != DType::BF16 || info.shape.size() != 2)
            return fail("quantize_checkpoint: " + e.first + " must be a 2-D BF16 weight");
        Tensor w = loader.load_tensor(e.first);
        QuantizedWeight qw = mode == QuantMode::INT8_HADAMARD ? quantize_weight_tensor(w) : quantize_weight_tensor_fp8(w);
        w.free_data();
        const int64_t N = info.shape[0], K = info.shape[1];
        std::vector<uint8_t> data(qw.data.nbytes());
        std::vector<uint8_t> scales(qw.scales.nbytes());
        qw.data.to_host(data.data());
        qw.scales.to_host(scales.data());
        qw.free_data();
        writer.add(e.first, qdt, {N, K}, data.data(), data.size());
        writer.add(e.first + ".__scales__", "F32", {N}, scales.data(), scales.size());
    }
    if (!writer.write(out)) return fail("failed to write " + out);
    return true;
}

// ---- C ABI -----------------------------------------------------------------
namespace {
int put_err(char* buf, int len, const std::string& m) {
    if (buf && len > 0) {
        const size_t n = m.size() < static_cast<size_t>(len - 1) ? m.size() : static_cast<size_t>(len - 1);
        memcpy(buf, m.data(), n);
        buf[n] = 0;
    }
    return -1;
}
}  // namespace

extern "C" {

void* qimg_st_writer_new(void) { return new (std::nothrow) SafeTensorsWriter(); }

int qimg_st_writer_add(void* w, const char* name, const char* dtype, const int64_t* shape, int ndim,
                       const void* data, size_t nbytes) {
    if (!w || !name || !dtype || ndim < 0 || (ndim > 0 && !shape) || (nbytes > 0 && !data)) return -1;
    static_cast<SafeTensorsWriter*>(w)->add(name, dtype, std::vector<int64_t>(shape, shape + ndim), data, nbytes);
    return 0;
}

int qimg_st_writer_write(void* w, const char* path) {
    if (!w || !path) return -1;
    return static_cast<SafeTensorsWriter*>(w)->write(path) ? 0 : -1;
}

void qimg_st_writer_free(void* w) { delete static_cast<SafeTensorsWriter*>(w); }

int qimg_checkpoint_kind(const char* path, char* err, int err_len) {
    if (!path) return put_err(err, err_len, "null path");
    SafeTensorsLoader loader;
    if (!load_model_dir(path, loader))
        return put_err(err, err_len, loader.error().empty() ? std::string("no safetensors checkpoint at ") + path
                                                            : loader.error());
    return static_cast<int>(detect_checkpoint(loader));
}

int qimg_quantize_checkpoint(const char* in_path, const char* out_path, int mode, int num_blocks, char* err,
                             int err_len) {
    if (!in_path || !out_path) return put_err(err, err_len, "null path");
    if (mode != QIMG_QM_INT8_HADAMARD && mode != QIMG_QM_FP8_HADAMARD)
        return put_err(err, err_len, "mode must be QIMG_QM_INT8_HADAMARD or QIMG_QM_FP8_HADAMARD");
    std::string m;
    const QuantMode qm = mode == QIMG_QM_INT8_HADAMARD ? QuantMode::INT8_HADAMARD : QuantMode::FP8_HADAMARD;
    if (!quantize_checkpoint(in_path, out_path, qm, num_blocks, &m)) return put_err(err, err_len, m);
    return 0;
}

}  // extern "C"
