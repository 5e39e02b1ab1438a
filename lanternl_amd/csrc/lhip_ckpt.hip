// lhip_ckpt.hip -- the LMTrain checkpoint format (lmio v3), written from and
// read into the flat parameter vector, on the host or straight from/to the
// device model.
//
// Format (ai/optim/lmio.lua:5-13,60-62,226-313,393-611):
//   "lanternl-checkpoint 3\n"
//   "format=bin|text dtype=f32 endian=le vocab=.. dim=.. layers=.. heads=..
//    ffn=.. pos=rope causal=0|1 tie=1 max_seq=.. rope_base=%g nparams=..
//    backend=.. epoch=.. loss=%.9g best_loss=%.9g [extra]\n"
//   per tensor in Transformer:parameters() order:
//     bin:  "<rows> <cols>\n" then rows*cols little-endian values
//     text: "<rows> <cols>|v,v,...\n" with %.9g (f32); nan / inf / -inf
// Readers also accept v2 (text, tag line) and v1 (no tag line, no "r c|"
// prefix), dtype f64 (converted to fp32) and CRLF line ends.  A write goes to
// "<path>.tmp<pid>" in the same directory, is closed with every write checked,
// then the older files rotate (path.(K-1) removed, path.i -> path.(i+1),
// path -> path.1 when keep = K > 1) and the temp file is renamed over path.
// Values stream through a fixed staging buffer (pinned when the device is
// the source), so memory does not grow with the model.
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "lhip_internal.h"

namespace lhip {
namespace {

constexpr const char* kTag = "lanternl-checkpoint";
constexpr int kVersion = 3;
constexpr long long kChunk = 1 << 20;   // values per staging pass

struct Tensor {
    long long off;
    int rows, cols;
};

std::vector<Tensor> tensors_of(const lhip_lm_config_t& c)
{
    const int nt = 2 + 9 * c.layers;
    std::vector<long long> off(nt);
    std::vector<int> rows(nt), cols(nt);
    lhip_lm_param_offsets(&c, off.data(), rows.data(), cols.data());
    std::vector<Tensor> t(nt);
    for (int i = 0; i < nt; ++i) t[i] = {off[i], rows[i], cols[i]};
    return t;
}

std::string fmt_num(double v, const char* prec)
{
    if (v != v) return "nan";
    if (v == HUGE_VAL) return "inf";
    if (v == -HUGE_VAL) return "-inf";
    char b[64];
    std::snprintf(b, sizeof b, prec, v);
    return b;
}

// Source of parameter values: fills dst[0..count) with elements
// [from, from+count) of the flat vector.
struct Source {
    const float* host = nullptr;      // host vector, or
    const float* dev = nullptr;       // device vector staged through `stage`
    float* stage = nullptr;
    int fetch(long long from, long long count, const float** out)
    {
        if (host) {
            *out = host + from;
            return LHIP_OK;
        }
        LHIP_CHECK_HIP(hipMemcpyAsync(stage, dev + from, static_cast<size_t>(count) * sizeof(float),
                                      hipMemcpyDeviceToHost, st().stream),
                       "checkpoint: device read");
        LHIP_CHECK_HIP(hipStreamSynchronize(st().stream), "checkpoint: sync");
        *out = stage;
        return LHIP_OK;
    }
};

struct Sink {
    float* host = nullptr;
    float* dev = nullptr;
    float* stage = nullptr;
    float* buffer(long long from) { return host ? host + from : stage; }
    int commit(long long from, long long count)
    {
        if (host) return LHIP_OK;
        LHIP_CHECK_HIP(hipMemcpyAsync(dev + from, stage, static_cast<size_t>(count) * sizeof(float),
                                      hipMemcpyHostToDevice, st().stream),
                       "checkpoint: device write");
        LHIP_CHECK_HIP(hipStreamSynchronize(st().stream), "checkpoint: sync");
        return LHIP_OK;
    }
};

int check_cfg(const lhip_lm_config_t* c, const char* who)
{
    if (!c) return fail(LHIP_E_NULL, "%s: config is NULL", who);
    if (c->vocab <= 0 || c->dim <= 0 || c->layers <= 0 || c->heads <= 0 || c->ffn <= 0)
        return fail(LHIP_E_SHAPE, "%s: every model size must be > 0", who);
    return LHIP_OK;
}

void rotate(const std::string& path, int keep)
{
    if (keep <= 1) return;
    std::remove((path + "." + std::to_string(keep - 1)).c_str());
    for (int i = keep - 2; i >= 1; --i)
        std::rename((path + "." + std::to_string(i)).c_str(), (path + "." + std::to_string(i + 1)).c_str());
    std::rename(path.c_str(), (path + ".1").c_str());
}

int write_checkpoint(const char* path, const lhip_lm_config_t& c, const lhip_ckpt_info_t* info, Source& src)
{
    if (!path || !*path) return fail(LHIP_E_ARG, "checkpoint save: expected a file path");
    const int text = info && info->format == 1;
    if (info && info->format != 0 && info->format != 1)
        return fail(LHIP_E_ARG, "checkpoint save: unknown format %d (0 = bin, 1 = text)", info->format);
    const std::vector<Tensor> ts = tensors_of(c);
    const std::string final_path(path);
    const std::string tmp = final_path + ".tmp" + std::to_string(static_cast<long long>(getpid()));
    FILE* f = std::fopen(tmp.c_str(), "wb");
    if (!f) return fail(LHIP_E_ARG, "checkpoint save: cannot write %s: %s", tmp.c_str(), std::strerror(errno));
    auto bail = [&](int code, const char* msg) {
        std::fclose(f);
        std::remove(tmp.c_str());
        return fail(code, "checkpoint save: %s (%s)", msg, tmp.c_str());
    };
    // header (lmio.lua:226-257)
    std::string h = std::string(kTag) + " " + std::to_string(kVersion) + "\n";
    char b[256];
    std::snprintf(b, sizeof b, "format=%s dtype=f32 endian=le vocab=%d dim=%d layers=%d heads=%d ffn=%d pos=rope "
                  "causal=%d tie=1 max_seq=%d", text ? "text" : "bin", c.vocab, c.dim, c.layers, c.heads, c.ffn,
                  c.causal ? 1 : 0, c.seq > 0 ? c.seq : 128);
    h += b;
    std::snprintf(b, sizeof b, " rope_base=%g nparams=%d", c.rope_base, static_cast<int>(ts.size()));
    h += b;
    h += " backend=";
    h += (info && info->backend) ? info->backend : "luatl_adapter";
    h += " epoch=" + std::to_string(info ? info->epoch : 0);
    h += " loss=" + (info && std::isfinite(info->loss) ? fmt_num(info->loss, "%.9g") : std::string("nan"));
    h += " best_loss=" +
         (info && std::isfinite(info->best_loss) ? fmt_num(info->best_loss, "%.9g") : std::string("nan"));
    if (info && info->extra && *info->extra) {
        h += " ";
        h += info->extra;
    }
    h += "\n";
    if (std::fwrite(h.data(), 1, h.size(), f) != h.size()) return bail(LHIP_E_ARG, "short write in header");
    // tensors (lmio.lua:259-313)
    std::string line;
    for (const Tensor& t : ts) {
        const long long total = static_cast<long long>(t.rows) * t.cols;
        std::snprintf(b, sizeof b, text ? "%d %d|" : "%d %d\n", t.rows, t.cols);
        if (std::fputs(b, f) < 0) return bail(LHIP_E_ARG, "short write");
        for (long long k = 0; k < total; k += kChunk) {
            const long long cn = std::min(kChunk, total - k);
            const float* vals = nullptr;
            if (int rc = src.fetch(t.off + k, cn, &vals)) {
                std::fclose(f);
                std::remove(tmp.c_str());
                return rc;
            }
            if (!text) {
                if (std::fwrite(vals, sizeof(float), static_cast<size_t>(cn), f) != static_cast<size_t>(cn))
                    return bail(LHIP_E_ARG, "short write (disk full?)");
            } else {
                line.clear();
                for (long long j = 0; j < cn; ++j) {
                    if (k + j > 0) line += ',';
                    line += fmt_num(vals[j], "%.9g");
                }
                if (std::fwrite(line.data(), 1, line.size(), f) != line.size())
                    return bail(LHIP_E_ARG, "short write (disk full?)");
            }
        }
        if (text && std::fputc('\n', f) == EOF) return bail(LHIP_E_ARG, "short write");
    }
    if (std::fclose(f) != 0) {
        std::remove(tmp.c_str());
        return fail(LHIP_E_ARG, "checkpoint save: close failed (disk full?): %s", std::strerror(errno));
    }
    rotate(final_path, info ? info->keep : 1);
    if (std::rename(tmp.c_str(), final_path.c_str()) != 0) {
        const int e = errno;
        std::remove(tmp.c_str());
        return fail(LHIP_E_ARG, "checkpoint save: rename %s -> %s failed: %s", tmp.c_str(), final_path.c_str(),
                    std::strerror(e));
    }
    return LHIP_OK;
}

// ---------------------------------------------------------------- reading
struct Reader {
    FILE* f = nullptr;
    ~Reader()
    {
        if (f) std::fclose(f);
    }
    // one line without its "\n" (and a trailing "\r"); false at EOF
    bool line(std::string& out)
    {
        out.clear();
        int ch;
        bool any = false;
        while ((ch = std::fgetc(f)) != EOF) {
            any = true;
            if (ch == '\n') break;
            out += static_cast<char>(ch);
        }
        if (!out.empty() && out.back() == '\r') out.pop_back();
        return any;
    }
};

bool field(const std::string& h, const char* key, std::string& val)
{
    const std::string k = std::string(key) + "=";
    size_t p = 0;
    while ((p = h.find(k, p)) != std::string::npos) {
        if (p == 0 || h[p - 1] == ' ') {
            const size_t e = h.find(' ', p);
            val = h.substr(p + k.size(), e == std::string::npos ? std::string::npos : e - p - k.size());
            return true;
        }
        p += k.size();
    }
    return false;
}

bool parse_num(const char* s, const char* e, double* out)
{
    std::string t(s, e);
    size_t a = 0, b = t.size();
    while (a < b && std::isspace(static_cast<unsigned char>(t[a]))) ++a;
    while (b > a && std::isspace(static_cast<unsigned char>(t[b - 1]))) --b;
    t = t.substr(a, b - a);
    if (t.empty()) return false;
    char* end = nullptr;
    const double v = std::strtod(t.c_str(), &end);   // also takes inf, -inf, nan (any case)
    if (end != t.c_str() + t.size()) return false;
    *out = v;
    return true;
}

int read_checkpoint(const char* path, const lhip_lm_config_t& c, Sink& sink, lhip_ckpt_header_t* hdr)
{
    if (!path || !*path) return fail(LHIP_E_ARG, "checkpoint load: expected a file path");
    Reader r;
    r.f = std::fopen(path, "rb");
    if (!r.f) return fail(LHIP_E_ARG, "checkpoint load: cannot open %s: %s", path, std::strerror(errno));
    std::string l1;
    if (!r.line(l1)) return fail(LHIP_E_ARG, "checkpoint load: %s is empty", path);
    bool legacy = true;
    int version = 1;
    std::string header = l1;
    const size_t tl = std::strlen(kTag);
    if (l1.compare(0, tl, kTag) == 0) {   // lmio.lua:426-441 (a plain prefix match)
        legacy = false;
        version = std::atoi(l1.c_str() + tl);
        if (version <= 0) version = 2;
        if (version > kVersion)
            return fail(LHIP_E_UNSUPPORTED, "checkpoint load: %s is format v%d, this build understands up to v%d",
                        path, version, kVersion);
        if (!r.line(header)) return fail(LHIP_E_ARG, "checkpoint load: %s is truncated (no header line)", path);
    }
    std::string v;
    int dims[5];
    const char* keys[5] = {"vocab", "dim", "layers", "heads", "ffn"};
    for (int i = 0; i < 5; ++i) {
        if (!field(header, keys[i], v)) return fail(LHIP_E_ARG, "checkpoint load: unrecognised header in %s", path);
        dims[i] = std::atoi(v.c_str());
    }
    const int want[5] = {c.vocab, c.dim, c.layers, c.heads, c.ffn};
    for (int i = 0; i < 5; ++i)
        if (dims[i] != want[i])
            return fail(LHIP_E_SHAPE, "checkpoint load: %s has %s=%d, the model has %d", path, keys[i], dims[i],
                        want[i]);
    const bool text = !field(header, "format", v) || v != "bin";
    const int es = (field(header, "dtype", v) ? v : std::string("f64")) == "f32" ? 4 : 8;
    if (!text && field(header, "endian", v) && v == "be")
        return fail(LHIP_E_UNSUPPORTED, "checkpoint load: endianness mismatch reading %s", path);
    lhip_ckpt_header_t hd{};
    hd.version = version;
    hd.format = text ? 1 : 0;
    hd.dtype_bytes = es;
    hd.epoch = -1;
    hd.loss = hd.best_loss = hd.rope_base = NAN;
    hd.causal = hd.tie = hd.max_seq = -1;
    if (!legacy) {
        if (field(header, "pos", v) && v != "rope")
            return fail(LHIP_E_UNSUPPORTED, "checkpoint load: pos=%s (this model uses RoPE)", v.c_str());
        if (field(header, "tie", v)) {
            hd.tie = std::atoi(v.c_str());
            if (hd.tie != 1)
                return fail(LHIP_E_UNSUPPORTED, "checkpoint load: untied head (tie=0) is not this model's layout");
        }
        if (field(header, "causal", v)) hd.causal = std::atoi(v.c_str());
        if (field(header, "max_seq", v)) hd.max_seq = std::atoi(v.c_str());
        if (field(header, "rope_base", v)) hd.rope_base = std::strtod(v.c_str(), nullptr);
        if (field(header, "epoch", v)) hd.epoch = std::atoi(v.c_str());
        double x;
        if (field(header, "loss", v) && parse_num(v.data(), v.data() + v.size(), &x)) hd.loss = x;
        if (field(header, "best_loss", v) && parse_num(v.data(), v.data() + v.size(), &x)) hd.best_loss = x;
    }
    const std::vector<Tensor> ts = tensors_of(c);
    if (field(header, "nparams", v) && std::atoi(v.c_str()) != static_cast<int>(ts.size()))
        return fail(LHIP_E_SHAPE, "checkpoint load: checkpoint has %d parameter tensors but this model has %d "
                    "(tie/arch mismatch?)", std::atoi(v.c_str()), static_cast<int>(ts.size()));
    std::vector<unsigned char> raw;
    for (size_t i = 0; i < ts.size(); ++i) {
        const Tensor& t = ts[i];
        const long long total = static_cast<long long>(t.rows) * t.cols;
        const int pi = static_cast<int>(i) + 1;
        if (!text) {
            std::string dl;
            if (!r.line(dl)) return fail(LHIP_E_ARG, "checkpoint load: %s is truncated at parameter %d", path, pi);
            int rr = -1, cc = -1;
            char tail = 0;
            if (std::sscanf(dl.c_str(), "%d %d%c", &rr, &cc, &tail) != 2 || rr != t.rows || cc != t.cols)
                return fail(LHIP_E_SHAPE, "checkpoint load: parameter %d is %s in the file but %dx%d in the model",
                            pi, dl.c_str(), t.rows, t.cols);
            for (long long k = 0; k < total; k += kChunk) {
                const long long cn = std::min(kChunk, total - k);
                raw.resize(static_cast<size_t>(cn) * es);
                if (std::fread(raw.data(), 1, raw.size(), r.f) != raw.size())
                    return fail(LHIP_E_ARG, "checkpoint load: %s is truncated inside parameter %d", path, pi);
                float* dst = sink.buffer(t.off + k);
                if (es == 4) {
                    std::memcpy(dst, raw.data(), raw.size());
                } else {
                    for (long long j = 0; j < cn; ++j) {
                        double d;
                        std::memcpy(&d, raw.data() + 8 * j, 8);
                        dst[j] = static_cast<float>(d);
                    }
                }
                if (int rc = sink.commit(t.off + k, cn)) return rc;
            }
        } else {
            std::string line;
            if (!r.line(line)) return fail(LHIP_E_ARG, "checkpoint load: %s is truncated at parameter %d", path, pi);
            const char* p = line.c_str();
            const char* end = p + line.size();
            if (!legacy) {
                const char* bar = static_cast<const char*>(std::memchr(p, '|', line.size()));
                int rr = -1, cc = -1;
                if (!bar || std::sscanf(p, "%d %d", &rr, &cc) != 2)
                    return fail(LHIP_E_ARG, "checkpoint load: malformed parameter line %d", pi);
                if (rr != t.rows || cc != t.cols)
                    return fail(LHIP_E_SHAPE, "checkpoint load: parameter %d is %dx%d in the file but %dx%d in the "
                                "model", pi, rr, cc, t.rows, t.cols);
                p = bar + 1;
            }
            long long j = 0, base = 0, fill = 0;
            float* dst = sink.buffer(t.off);
            while (p < end) {
                const char* q = static_cast<const char*>(std::memchr(p, ',', static_cast<size_t>(end - p)));
                if (!q) q = end;
                if (q > p) {   // empty fields are skipped, as gmatch("[^,]+") does
                    if (j >= total) {
                        ++j;
                        break;
                    }
                    double x;
                    if (!parse_num(p, q, &x))
                        return fail(LHIP_E_ARG, "checkpoint load: parameter %d value %lld is not a number ('%s')", pi,
                                    j + 1, std::string(p, q).c_str());
                    dst[fill++] = static_cast<float>(x);
                    ++j;
                    if (fill == kChunk) {
                        if (int rc = sink.commit(t.off + base, fill)) return rc;
                        base += fill;
                        fill = 0;
                        dst = sink.buffer(t.off + base);
                    }
                }
                p = q + 1;
            }
            if (fill > 0)
                if (int rc = sink.commit(t.off + base, fill)) return rc;
            if (j != total)
                return fail(LHIP_E_SHAPE, "checkpoint load: parameter %d has %lld values, expected %lld", pi, j, total);
        }
    }
    if (hdr) *hdr = hd;
    return LHIP_OK;
}

}  // namespace
}  // namespace lhip

using lhip::fail;
using lhip::st;

extern "C" {

LHIP_API int lhip_ckpt_save_host(const char* path, const lhip_lm_config_t* cfg, const lhip_ckpt_info_t* info,
                                 const float* params, long long n)
{
    if (int rc = lhip::check_cfg(cfg, "lhip_ckpt_save_host")) return rc;
    if (!params) return fail(LHIP_E_NULL, "lhip_ckpt_save_host: params is NULL");
    if (n != lhip_lm_num_params(cfg))
        return fail(LHIP_E_SHAPE, "lhip_ckpt_save_host: %lld values given, model has %lld", n, lhip_lm_num_params(cfg));
    lhip::Source src;
    src.host = params;
    return lhip::write_checkpoint(path, *cfg, info, src);
}

LHIP_API int lhip_ckpt_load_host(const char* path, const lhip_lm_config_t* cfg, float* params, long long n,
                                 lhip_ckpt_header_t* header)
{
    if (int rc = lhip::check_cfg(cfg, "lhip_ckpt_load_host")) return rc;
    if (!params) return fail(LHIP_E_NULL, "lhip_ckpt_load_host: params is NULL");
    if (n != lhip_lm_num_params(cfg))
        return fail(LHIP_E_SHAPE, "lhip_ckpt_load_host: %lld values given, model has %lld", n, lhip_lm_num_params(cfg));
    lhip::Sink sink;
    sink.host = params;
    return lhip::read_checkpoint(path, *cfg, sink, header);
}

}  // extern "C"

// Device-model save/load: the parameter vector streams through one pinned
// staging buffer of kChunk floats.
namespace lhip {

int lm_checkpoint_io(const lhip_lm_config_t& cfg, float* dev_params, const char* path, const lhip_ckpt_info_t* info,
                     lhip_ckpt_header_t* header, bool save)
{
    float* stage = nullptr;
    LHIP_CHECK_HIP(hipHostMalloc(reinterpret_cast<void**>(&stage), kChunk * sizeof(float), hipHostMallocDefault),
                   "checkpoint: pinned staging");
    LHIP_CHECK_HIP(hipStreamSynchronize(st().stream), "checkpoint: sync");
    int rc;
    if (save) {
        Source src;
        src.dev = dev_params;
        src.stage = stage;
        rc = write_checkpoint(path, cfg, info, src);
    } else {
        Sink sink;
        sink.dev = dev_params;
        sink.stage = stage;
        rc = read_checkpoint(path, cfg, sink, header);
    }
    (void)hipHostFree(stage);
    return rc;
}

}  // namespace lhip
