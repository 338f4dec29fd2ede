// serve.cpp -- the serve-directory protocol (the reference's persistent `--serve DIR` loop,
// hpc_gpu_port/gpu_real_model.cu:4363-4483 for the wait/request side and :5525-5576 for the answer; the client side
// is ml-eval/fhe_client.py:1394-1492, serve_roundtrip).  Host code only: the request's computation is a handler
// (fhe_ssm_decoder_serve passes the decode step's), so the file protocol runs and is tested without a GPU.
//
// Inside DIR, request N (N counts from 0 per server):
//   client  writes req.N.0 .. req.N.<count-1> and req.N.meta (one-line JSON with integer values), optionally
//           req.N.reset (drop the carried state first), then req.N.ready LAST
//   server  writes serve.status {"nextReq","served","pid","stateful","storeFile"} (tmp + rename) while waiting,
//           polls for `stop` or req.N.ready, reads the meta (unreadable, tokensReal < 1 or count outside
//           [1, 65536]: resp.N.error, the
//           ready marker removed, next N), runs the handler, touches resp.N.done (or resp.N.error), and only then
//           removes req.N.<t>, req.N.meta and req.N.ready -- the client's completion test is "done and not ready".
//   exit    a file named `stop`, or timeout_sec idle seconds with no request.
// Log lines are one JSON object each: serve = waiting | request | stateReset | badRequest | served | exit.
#include <sys/stat.h>
#include <unistd.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>
#include <thread>

#include "fhe_ssm_decode.h"

namespace fhe_ssm_detail {
void set_error(const std::string& m);  // host/decode.cpp
}  // namespace fhe_ssm_detail

namespace {

using Clock = std::chrono::steady_clock;
constexpr long long kMaxCount = 1 << 16;  // ciphertext files per request

bool exists(const std::string& p) { return ::access(p.c_str(), F_OK) == 0; }

bool is_dir(const std::string& p) {
    struct stat st;
    return ::stat(p.c_str(), &st) == 0 && S_ISDIR(st.st_mode);
}

void touch(const std::string& p, const char* msg) {
    std::ofstream f(p);
    f << msg << "\n";
}

bool read_text(const std::string& p, std::string* out) {
    std::ifstream f(p);
    if (!f) return false;
    std::stringstream ss;
    ss << f.rdbuf();
    *out = ss.str();
    return true;
}

void log_line(int fd, const std::string& s) {
    if (fd < 0) return;
    const std::string line = s + "\n";
    size_t off = 0;
    while (off < line.size()) {
        const ssize_t w = ::write(fd, line.data() + off, line.size() - off);
        if (w <= 0) return;
        off += (size_t)w;
    }
}

// a JSON string literal: quote and backslash escaped, control characters as \u00XX
std::string q(const std::string& s) {
    std::string o = "\"";
    for (char c : s) {
        if (c == '"' || c == '\\') {
            o += '\\';
            o += c;
        } else if ((unsigned char)c < 0x20) {
            char buf[8];
            std::snprintf(buf, sizeof buf, "\\u%04x", (unsigned)(unsigned char)c);
            o += buf;
        } else {
            o += c;
        }
    }
    return o + "\"";
}

}  // namespace

extern "C" {

// The meta sidecar is a flat one-line JSON object whose values are integers, written and read by the two ends of
// the protocol; a key is found by its quoted name followed by a colon (the reference's metaInt,
// gpu_real_model.cu:2327-2331).  Absent keys give dflt.
long long fhe_ssm_meta_int(const char* text, const char* key, long long dflt) {
    if (!text || !key) return dflt;
    const std::string t(text), k = std::string("\"") + key + "\":";
    const size_t pos = t.find(k);
    if (pos == std::string::npos) return dflt;
    return std::atoll(t.c_str() + pos + k.size());
}

int fhe_ssm_serve_dir(const char* dir, const fhe_ssm_serve_opts* opts, fhe_ssm_serve_handler handler, void* user,
                      fhe_ssm_serve_report* report) {
    if (!dir || !opts || !handler || !report) {
        fhe_ssm_detail::set_error("serve: null argument");
        return CKKS_EINVAL;
    }
    const std::string D(dir);
    if (!is_dir(D)) {
        fhe_ssm_detail::set_error("serve: " + D + " is not a directory");
        return CKKS_EINVAL;
    }
    const int fd = opts->log_fd;
    const uint32_t poll_ms = opts->poll_ms ? opts->poll_ms : 200;
    std::memset(report, 0, sizeof(*report));
    uint32_t n = opts->first_req, served = 0, failed = 0;
    for (;;) {
        const std::string req = D + "/req." + std::to_string(n), resp = D + "/resp." + std::to_string(n);
        log_line(fd, "{\"serve\":\"waiting\",\"req\":" + std::to_string(n) + ",\"dir\":" + q(D) +
                         ",\"timeoutSec\":" + std::to_string(opts->timeout_sec) +
                         ",\"served\":" + std::to_string(served) + "}");
        {
            std::ofstream sf(D + "/serve.status.tmp");
            sf << "{\"nextReq\":" << n << ",\"served\":" << served << ",\"pid\":" << (long long)getpid()
               << ",\"stateful\":" << (opts->stateful ? "true" : "false") << ",\"storeFile\":\"\"}\n";
            sf.close();
            std::rename((D + "/serve.status.tmp").c_str(), (D + "/serve.status").c_str());
        }
        const auto t_wait = Clock::now();
        bool got_req = false, got_stop = false;
        for (;;) {
            if (exists(D + "/stop")) {
                got_stop = true;
                break;
            }
            if (exists(req + ".ready")) {
                got_req = true;
                break;
            }
            const double idle = std::chrono::duration<double>(Clock::now() - t_wait).count();
            if (idle > (double)opts->timeout_sec) break;
            std::this_thread::sleep_for(std::chrono::milliseconds(poll_ms));
        }
        if (!got_req) {
            report->exit_reason = got_stop ? 0 : 1;
            report->served = served;
            report->failed = failed;
            report->next_req = n;
            log_line(fd, std::string("{\"serve\":\"exit\",\"reason\":\"") + (got_stop ? "stop" : "idleTimeout") +
                             "\",\"served\":" + std::to_string(served) + "}");
            return CKKS_OK;
        }
        std::string meta;
        const bool have_meta = read_text(req + ".meta", &meta);
        const long long tokens = have_meta ? fhe_ssm_meta_int(meta.c_str(), "tokensReal", -1) : -1;
        const long long count = have_meta ? fhe_ssm_meta_int(meta.c_str(), "count", -1) : -1;
        if (tokens < 1 || count < 1 || count > kMaxCount) {
            log_line(fd, "{\"serve\":\"badRequest\",\"req\":" + std::to_string(n) + "}");
            touch(resp + ".error", "bad or missing request meta");
            std::remove((req + ".ready").c_str());
            failed++;
            n++;
            continue;
        }
        int reset = 0;
        if (exists(req + ".reset")) {
            reset = 1;
            std::remove((req + ".reset").c_str());
            log_line(fd, "{\"serve\":\"stateReset\",\"req\":" + std::to_string(n) + "}");
        }
        if (!opts->stateful) reset = 1;  // a stateless server starts every request from a cold state
        log_line(fd, "{\"serve\":\"request\",\"req\":" + std::to_string(n) + ",\"tokens\":" + std::to_string(tokens) + "}");
        const auto t0 = Clock::now();
        char err[512] = {0};
        const int rc = handler(user, n, req.c_str(), resp.c_str(), meta.c_str(), reset, err, sizeof err);
        err[sizeof err - 1] = 0;
        const double ms = std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
        // answer first, then remove the request files, the ready marker last
        if (rc != 0) {
            failed++;
            touch(resp + ".error", "forward failed; see the server log");
        } else {
            touch(resp + ".done", "ok");
        }
        for (long long i = 0; i < count; i++) std::remove((req + "." + std::to_string(i)).c_str());
        std::remove((req + ".meta").c_str());
        std::remove((req + ".ready").c_str());
        char buf[96];
        std::snprintf(buf, sizeof buf, "%.1f", ms / (double)tokens);
        log_line(fd, "{\"serve\":\"served\",\"req\":" + std::to_string(n) + ",\"failed\":" +
                         (rc != 0 ? "true" : "false") + ",\"tokens\":" + std::to_string(tokens) +
                         ",\"reqMs\":" + std::to_string((long long)ms) + ",\"reqMsPerToken\":" + buf +
                         (rc != 0 ? ",\"error\":" + q(err) : std::string()) + "}");
        served++;
        n++;
    }
}

}  // extern "C"
