// safetensors reading and checkpoint validation; see weights.h.
#include "weights.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstring>
#include <memory>
#include <set>
#include <sstream>

namespace scunet {
namespace {

// A minimal JSON value: enough for a safetensors header (objects, arrays, strings,
// integers, and the literals).
struct JVal {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    double num = 0;
    std::string str;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;
    const JVal* get(const std::string& k) const {
        for (auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

struct JParser {
    const char* p;
    const char* end;
    std::string err;
    void ws() {
        while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
    }
    bool fail(const char* m) {
        if (err.empty()) err = m;
        return false;
    }
    bool str(std::string* out) {
        if (p >= end || *p != '"') return fail("expected a string");
        ++p;
        while (p < end && *p != '"') {
            if (*p == '\\') {
                ++p;
                if (p >= end) return fail("bad escape");
                char c = *p++;
                switch (c) {
                    case 'n': out->push_back('\n'); break;
                    case 't': out->push_back('\t'); break;
                    case 'r': out->push_back('\r'); break;
                    case 'b': out->push_back('\b'); break;
                    case 'f': out->push_back('\f'); break;
                    case 'u': {
                        if (end - p < 4) return fail("bad \\u escape");
                        unsigned v = 0;
                        for (int i = 0; i < 4; ++i) {
                            char h = *p++;
                            v <<= 4;
                            if (h >= '0' && h <= '9') v |= unsigned(h - '0');
                            else if (h >= 'a' && h <= 'f') v |= unsigned(h - 'a' + 10);
                            else if (h >= 'A' && h <= 'F') v |= unsigned(h - 'A' + 10);
                            else return fail("bad \\u escape");
                        }
                        if (v < 0x80) out->push_back(char(v));
                        else if (v < 0x800) {
                            out->push_back(char(0xC0 | (v >> 6)));
                            out->push_back(char(0x80 | (v & 0x3F)));
                        } else {
                            out->push_back(char(0xE0 | (v >> 12)));
                            out->push_back(char(0x80 | ((v >> 6) & 0x3F)));
                            out->push_back(char(0x80 | (v & 0x3F)));
                        }
                        break;
                    }
                    default: out->push_back(c);
                }
            } else {
                out->push_back(*p++);
            }
        }
        if (p >= end) return fail("unterminated string");
        ++p;
        return true;
    }
    bool val(JVal* v, int depth) {
        if (depth > 16) return fail("nesting too deep");
        ws();
        if (p >= end) return fail("unexpected end");
        char c = *p;
        if (c == '{') {
            v->kind = JVal::OBJ;
            ++p;
            ws();
            if (p < end && *p == '}') { ++p; return true; }
            while (true) {
                ws();
                std::string k;
                if (!str(&k)) return false;
                ws();
                if (p >= end || *p != ':') return fail("expected ':'");
                ++p;
                JVal x;
                if (!val(&x, depth + 1)) return false;
                v->obj.emplace_back(std::move(k), std::move(x));
                ws();
                if (p < end && *p == ',') { ++p; continue; }
                if (p < end && *p == '}') { ++p; return true; }
                return fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            v->kind = JVal::ARR;
            ++p;
            ws();
            if (p < end && *p == ']') { ++p; return true; }
            while (true) {
                JVal x;
                if (!val(&x, depth + 1)) return false;
                v->arr.push_back(std::move(x));
                ws();
                if (p < end && *p == ',') { ++p; continue; }
                if (p < end && *p == ']') { ++p; return true; }
                return fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v->kind = JVal::STR;
            return str(&v->str);
        }
        if (c == 't' && end - p >= 4 && !std::strncmp(p, "true", 4)) { v->kind = JVal::BOOL; v->num = 1; p += 4; return true; }
        if (c == 'f' && end - p >= 5 && !std::strncmp(p, "false", 5)) { v->kind = JVal::BOOL; p += 5; return true; }
        if (c == 'n' && end - p >= 4 && !std::strncmp(p, "null", 4)) { v->kind = JVal::NUL; p += 4; return true; }
        if (c == '-' || (c >= '0' && c <= '9')) {
            const char* s = p;
            while (p < end && (*p == '-' || *p == '+' || *p == '.' || *p == 'e' || *p == 'E' ||
                               (*p >= '0' && *p <= '9')))
                ++p;
            v->kind = JVal::NUM;
            v->num = std::strtod(std::string(s, p).c_str(), nullptr);
            return true;
        }
        return fail("unexpected character");
    }
};

std::string shape_str(const std::vector<size_t>& s) {
    std::ostringstream o;
    o << "[";
    for (size_t i = 0; i < s.size(); ++i) o << (i ? ", " : "") << s[i];
    o << "]";
    return o.str();
}

// A JSON number that is an integer in [0, max].
bool whole(const JVal& v, double max) {
    return v.kind == JVal::NUM && std::isfinite(v.num) && v.num >= 0 && v.num <= max && v.num == std::floor(v.num);
}

// weights.rs:44-60 / 76-81: the eight published variants and their in_nc.
int variant_in_nc(const std::string& v) {
    static const char* color[] = {"color-15", "color-25", "color-50", "color-real-psnr", "color-real-gan"};
    static const char* gray[] = {"gray-15", "gray-25", "gray-50"};
    for (auto c : color)
        if (v == c) return 3;
    for (auto g : gray)
        if (v == g) return 1;
    return -1;
}

const char* STAGE[7] = {"down1", "down2", "down3", "body", "up3", "up2", "up1"};

}  // namespace

Weights::~Weights() {
    if (map_) munmap(map_, map_len_);
}

const Tensor& Weights::t(const std::string& name) const {
    auto it = t_.find(name);
    if (it == t_.end()) {
        static Tensor empty;
        return empty;
    }
    return it->second;
}

std::pair<int, int> Weights::block_dims(const std::string& prefix) const {
    int total = int(t(prefix + ".conv1_1.weight").shape.at(0));
    int trans = int(t(prefix + ".trans_block.msa.linear.weight").shape.at(0));
    return {total - trans, trans};
}

std::pair<int, int> Weights::up_conv_channels(const std::string& name) const {
    auto d = block_dims("m_" + name + ".1");
    return {2 * (d.first + d.second), d.first + d.second};
}

std::pair<int, int> Weights::down_conv_channels(const std::string& name) const {
    int count = name == "down1" ? config[0] : name == "down2" ? config[1] : config[2];
    auto d = block_dims("m_" + name + "." + std::to_string(count - 1));
    return {d.first + d.second, 2 * (d.first + d.second)};
}

bool Weights::load(const std::string& path, std::string* err) {
    int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) {
        *err = path + ": " + std::strerror(errno);
        return false;
    }
    struct stat st;
    if (fstat(fd, &st) != 0) {
        *err = path + ": " + std::strerror(errno);
        ::close(fd);
        return false;
    }
    map_len_ = size_t(st.st_size);
    bytes = uint64_t(st.st_size);
    if (map_len_ < 8) {
        *err = path + ": too short to be a safetensors file";
        ::close(fd);
        return false;
    }
    map_ = mmap(nullptr, map_len_, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (map_ == MAP_FAILED) {
        map_ = nullptr;
        *err = path + ": mmap: " + std::strerror(errno);
        return false;
    }
    const uint8_t* base = static_cast<const uint8_t*>(map_);
    uint64_t hlen = 0;
    std::memcpy(&hlen, base, 8);
    if (hlen > map_len_ - 8) {
        *err = path + ": header length " + std::to_string(hlen) + " exceeds the file";
        return false;
    }
    JParser jp{reinterpret_cast<const char*>(base + 8), reinterpret_cast<const char*>(base + 8 + hlen), ""};
    JVal root;
    if (!jp.val(&root, 0) || root.kind != JVal::OBJ) {
        *err = path + ": header is not a JSON object (" + jp.err + ")";
        return false;
    }
    const uint8_t* data = base + 8 + hlen;
    size_t data_len = map_len_ - 8 - size_t(hlen);
    std::map<std::string, std::string> meta;
    for (auto& kv : root.obj) {
        if (kv.first == "__metadata__") {
            for (auto& m : kv.second.obj)
                if (m.second.kind == JVal::STR) meta[m.first] = m.second.str;
            continue;
        }
        const JVal* dt = kv.second.get("dtype");
        const JVal* sh = kv.second.get("shape");
        const JVal* off = kv.second.get("data_offsets");
        if (!dt || !sh || !off || off->arr.size() != 2) {
            *err = path + ": " + kv.first + ": malformed header entry";
            return false;
        }
        if (dt->str != "F32") {
            *err = path + ": " + kv.first + ": dtype " + dt->str + " is not F32";
            return false;
        }
        Tensor tt;
        size_t n = 1;
        for (auto& d : sh->arr) {
            // Extents are integers in [0, 2^32]; the element count may not overflow.
            if (!whole(d, 4294967296.0)) {
                *err = path + ": " + kv.first + ": shape entry is not an integer in [0, 2^32]";
                return false;
            }
            const size_t e = size_t(d.num);
            if (e != 0 && n > (SIZE_MAX / 4) / e) {
                *err = path + ": " + kv.first + ": shape " + shape_str(tt.shape) + " overflows";
                return false;
            }
            tt.shape.push_back(e);
            n *= e;
        }
        if (!whole(off->arr[0], 9007199254740992.0) || !whole(off->arr[1], 9007199254740992.0)) {
            *err = path + ": " + kv.first + ": data offsets are not non-negative integers";
            return false;
        }
        size_t a = size_t(off->arr[0].num), b = size_t(off->arr[1].num);
        if (b < a || b > data_len || b - a != n * 4) {
            *err = path + ": " + kv.first + ": data offsets disagree with its shape";
            return false;
        }
        if ((a & 3) != 0) {
            *err = path + ": " + kv.first + ": data is not 4-byte aligned";
            return false;
        }
        tt.data = reinterpret_cast<const float*>(data + a);
        tt.numel = n;
        t_[kv.first] = tt;
    }
    // weights.rs:116-126: the seven keys.
    for (const char* k : {"arch", "variant", "in_nc", "dim", "config", "head_dim", "window_size"}) {
        if (!meta.count(k)) {
            *err = path + ": no `" + k +
                   "` in __metadata__ - convert the checkpoint with tools/convert.py, which "
                   "records the architecture; a plain state_dict cannot be checked";
            return false;
        }
    }
    if (meta["arch"] != "scunet") {
        *err = path + ": __metadata__ says arch = \"" + meta["arch"] +
               "\", not `scunet` - this is a checkpoint for a different engine";
        return false;
    }
    auto num = [&](const char* k, int* out) {
        char* e = nullptr;
        long v = std::strtol(meta[k].c_str(), &e, 10);
        if (!e || *e != 0 || meta[k].empty() || v < 0) {
            *err = path + ": `" + k + "` = \"" + meta[k] + "\": not a non-negative integer";
            return false;
        }
        *out = int(v);
        return true;
    };
    {
        std::vector<int> cfg;
        std::stringstream ss(meta["config"]);
        std::string item;
        while (std::getline(ss, item, ',')) {
            char* e = nullptr;
            long v = std::strtol(item.c_str(), &e, 10);
            if (item.empty() || (e && *e != 0 && *e != ' ')) {
                *err = "config: invalid digit in \"" + item + "\"";
                return false;
            }
            cfg.push_back(int(v));
        }
        if (cfg.size() != 7) {
            *err = path + ": config has " + std::to_string(cfg.size()) +
                   " entries, SCUNet's seven stages need 7";
            return false;
        }
        for (int i = 0; i < 7; ++i) config[i] = cfg[size_t(i)];
    }
    // The order of weights.rs:127-160: the variant, in_nc against it, then the widths.
    variant = meta["variant"];
    if (variant_in_nc(variant) < 0) return check_arch(path, err);
    if (!num("in_nc", &in_nc)) return false;
    if (in_nc != variant_in_nc(variant)) return check_arch(path, err);
    if (!num("dim", &dim) || !num("head_dim", &head_dim) || !num("window_size", &window)) return false;
    if (!check_arch(path, err)) return false;
    return validate(path, err);
}

// The architecture checks of weights.rs:127-160 (variant, its in_nc, dim against head_dim).
bool Weights::check_arch(const std::string& label, std::string* err) const {
    int want_nc = variant_in_nc(variant);
    if (want_nc < 0) {
        *err = "variant `" + variant +
               "` is not one of the eight published SCUNet checkpoints (color-15, color-25, "
               "color-50, color-real-psnr, color-real-gan, gray-15, gray-25, gray-50)";
        return false;
    }
    if (in_nc != want_nc) {
        *err = label + ": variant " + variant + " implies in_nc " + std::to_string(want_nc) +
               ", the header says " + std::to_string(in_nc);
        return false;
    }
    if (head_dim == 0 || dim % head_dim != 0) {
        *err = label + ": dim " + std::to_string(dim) + " is not a multiple of head_dim " +
               std::to_string(head_dim);
        return false;
    }
    return true;
}

// Every tensor name the walker can ask for under this config: the head and tail, each
// stage's blocks (up stages number theirs from 1), the up-convolutions (m_upN.0) and the
// down-convolutions (m_downN.<count>).
std::vector<std::string> Weights::expected_names() const {
    std::vector<std::string> r = {"m_head.0.weight", "m_tail.0.weight"};
    static const char* BLOCK[] = {
        "conv1_1.weight", "conv1_1.bias", "conv1_2.weight", "conv1_2.bias", "conv_block.0.weight",
        "conv_block.2.weight", "trans_block.ln1.weight", "trans_block.ln1.bias", "trans_block.ln2.weight",
        "trans_block.ln2.bias", "trans_block.mlp.0.weight", "trans_block.mlp.0.bias",
        "trans_block.mlp.2.weight", "trans_block.mlp.2.bias", "trans_block.msa.embedding_layer.weight",
        "trans_block.msa.embedding_layer.bias", "trans_block.msa.linear.weight",
        "trans_block.msa.linear.bias", "trans_block.msa.relative_position_params"};
    for (int stage = 0; stage < 7; ++stage) {
        const std::string m = "m_" + std::string(STAGE[stage]) + ".";
        const int first = stage >= 4 ? 1 : 0;
        for (int b = first; b < first + config[stage]; ++b)
            for (const char* k : BLOCK) r.push_back(m + std::to_string(b) + "." + k);
        if (stage >= 4) r.push_back(m + "0.weight");
        if (stage < 3) r.push_back(m + std::to_string(config[stage]) + ".weight");
    }
    return r;
}

bool Weights::borrow(const ArchInfo& a, TensorLookup lookup, void* user, std::string* err) {
    const std::string label = "weights";
    if (!lookup) {
        *err = label + ": no tensor lookup given";
        return false;
    }
    auto fits = [](long v) { return v >= 0 && v <= 1 << 20; };
    if (!fits(a.in_nc) || !fits(a.dim) || !fits(a.head_dim) || !fits(a.window)) {
        *err = label + ": in_nc, dim, head_dim and window must be integers in [0, 2^20]";
        return false;
    }
    for (int i = 0; i < 7; ++i)
        if (a.config[i] < 1 || a.config[i] > 1024) {
            *err = label + ": config[" + std::to_string(i) + "] = " + std::to_string(a.config[i]) +
                   ": every stage needs between 1 and 1024 blocks";
            return false;
        }
    variant = a.variant;
    in_nc = int(a.in_nc);
    dim = int(a.dim);
    head_dim = int(a.head_dim);
    window = int(a.window);
    for (int i = 0; i < 7; ++i) config[i] = int(a.config[i]);
    if (!check_arch(label, err)) return false;
    t_.clear();
    for (const std::string& n : expected_names()) {
        size_t shape[MAX_NDIM] = {}, ndim = 0;
        const float* p = lookup(user, n.c_str(), shape, &ndim);
        if (!p) continue;   // validate() names the first missing tensor
        if (ndim > MAX_NDIM) {
            *err = label + ": " + n + ": more than " + std::to_string(MAX_NDIM) + " dimensions";
            return false;
        }
        Tensor tt;
        size_t count = 1;
        for (size_t i = 0; i < ndim; ++i) {
            if (shape[i] > (size_t(1) << 32) || (shape[i] != 0 && count > (SIZE_MAX / 4) / shape[i])) {
                *err = label + ": " + n + ": shape overflows";
                return false;
            }
            tt.shape.push_back(shape[i]);
            count *= shape[i];
        }
        tt.data = p;
        tt.numel = count;
        t_[n] = tt;
    }
    return validate(label, err);
}

void Weights::forget_data() {
    for (auto& kv : t_) kv.second.data = nullptr;
}

// weights.rs:204-280: every shape the walker will ask for. Tensors outside that list are
// dropped, so nothing unchecked is uploaded.
bool Weights::validate(const std::string& path, std::string* err) {
    std::vector<std::pair<std::string, std::vector<size_t>>> want;
    size_t d = size_t(dim), nc = size_t(in_nc), ws = size_t(window);
    want.push_back({"m_head.0.weight", {d, nc, 3, 3}});
    want.push_back({"m_tail.0.weight", {nc, d, 3, 3}});
    auto present = [&](const std::string& n) -> bool {
        if (!has(n)) {
            *err = path + ": " + n + ": no such tensor";
            return false;
        }
        return true;
    };
    for (int stage = 0; stage < 7; ++stage) {
        std::string name = STAGE[stage];
        int count = config[stage];
        int first = stage >= 4 ? 1 : 0;
        bool tail = stage < 3;
        if (first == 1) {
            std::string p1 = "m_" + name + ".1";
            if (!present(p1 + ".conv1_1.weight") || !present(p1 + ".trans_block.msa.linear.weight"))
                return false;
            auto ch = up_conv_channels(name);
            want.push_back({"m_" + name + ".0.weight", {size_t(ch.first), size_t(ch.second), 2, 2}});
        }
        for (int b = first; b < first + count; ++b) {
            std::string p = "m_" + name + "." + std::to_string(b);
            if (!present(p + ".conv1_1.weight") || !present(p + ".trans_block.msa.linear.weight"))
                return false;
            if (t(p + ".conv1_1.weight").shape.empty() || t(p + ".trans_block.msa.linear.weight").shape.empty()) {
                *err = path + ": " + p + ": scalar weight";
                return false;
            }
            auto dims = block_dims(p);
            size_t conv = size_t(dims.first), trans = size_t(dims.second), c = conv + trans;
            want.push_back({p + ".conv1_1.weight", {c, c, 1, 1}});
            want.push_back({p + ".conv1_1.bias", {c}});
            want.push_back({p + ".conv1_2.weight", {c, c, 1, 1}});
            want.push_back({p + ".conv1_2.bias", {c}});
            want.push_back({p + ".conv_block.0.weight", {conv, conv, 3, 3}});
            want.push_back({p + ".conv_block.2.weight", {conv, conv, 3, 3}});
            for (const char* k : {"ln1.weight", "ln1.bias", "ln2.weight", "ln2.bias"})
                want.push_back({p + ".trans_block." + k, {trans}});
            want.push_back({p + ".trans_block.mlp.0.weight", {4 * trans, trans}});
            want.push_back({p + ".trans_block.mlp.0.bias", {4 * trans}});
            want.push_back({p + ".trans_block.mlp.2.weight", {trans, 4 * trans}});
            want.push_back({p + ".trans_block.mlp.2.bias", {trans}});
            want.push_back({p + ".trans_block.msa.embedding_layer.weight", {3 * trans, trans}});
            want.push_back({p + ".trans_block.msa.embedding_layer.bias", {3 * trans}});
            want.push_back({p + ".trans_block.msa.linear.weight", {trans, trans}});
            want.push_back({p + ".trans_block.msa.linear.bias", {trans}});
            size_t heads = trans / size_t(head_dim);
            want.push_back({p + ".trans_block.msa.relative_position_params", {heads, 2 * ws - 1, 2 * ws - 1}});
        }
        if (tail) {
            std::string last = "m_" + name + "." + std::to_string(count - 1);
            if (!present(last + ".conv1_1.weight") || !present(last + ".trans_block.msa.linear.weight"))
                return false;
            auto ch = down_conv_channels(name);
            want.push_back({"m_" + name + "." + std::to_string(count) + ".weight",
                            {size_t(ch.second), size_t(ch.first), 2, 2}});
        }
    }
    std::set<std::string> checked;
    for (auto& w : want) {
        if (!present(w.first)) return false;
        const auto& got = t(w.first).shape;
        if (got != w.second) {
            *err = path + ": " + w.first + " is " + shape_str(got) + ", the " + std::to_string(dim) +
                   "-wide/" + std::to_string(window) + "-window/" + std::to_string(in_nc) +
                   "-channel architecture in the header implies " + shape_str(w.second);
            return false;
        }
        checked.insert(w.first);
    }
    for (auto it = t_.begin(); it != t_.end();) it = checked.count(it->first) ? std::next(it) : t_.erase(it);
    return true;
}

}  // namespace scunet
