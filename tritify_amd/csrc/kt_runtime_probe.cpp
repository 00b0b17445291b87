// kt_runtime_probe: probe a host as kt-runtime's runtime_probe does (crates/02-runtime/kt-runtime/examples/
// runtime_probe.rs:19-89) for this build's backends: what the host offers, whether every backend returns the same
// bytes on the fixed corpus (one SHA-256 each), whether each holds residency and the bound cases, and how fast each
// is on an OLMoE-sized projection. Exits 1 if any backend diverges.
//
//   tritify_amd/kt_runtime_probe [--budget-1] [--plants] [--no-speed]
//
// --budget-1 adds the device backend with a 1-byte budget (it evicts on every call). --plants loads the planted
// test build (libkt_hip_planted.so) and requires each planted defect to be caught, as kt-runtime's
// every_planted_digit_defect_is_caught does (src/tests_cuda.rs:47-72): DropPlane22 and WrongCarry by the equality
// gate, NoFlush by a bound case (the corpus never reaches the bound), CacheByShape by the residency gate.
//
// Both libraries are opened with dlopen and called through the C ABI of include/kt_hip.h.
#include <dlfcn.h>
#include <limits.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <sys/utsname.h>
#include <unistd.h>

#include <chrono>
#include <string>
#include <thread>
#include <vector>

#include "kt_hip.h"

namespace {

struct Lib {
    void* h = nullptr;
    decltype(&kt_hip_device_count) device_count;
    decltype(&kt_hip_device_info) device_info;
    decltype(&kt_hip_open) open;
    decltype(&kt_hip_open_planted) open_planted;
    decltype(&kt_hip_close) close;
    decltype(&kt_hip_linear) linear;
    decltype(&kt_hip_linear_weights) linear_weights;
    decltype(&kt_hip_weight_id_fresh) weight_id_fresh;
    decltype(&kt_hip_fallbacks) fallbacks;
    decltype(&kt_hip_error_string) error_string;
    decltype(&kt_hip_gate_corpus) gate_corpus;
    decltype(&kt_hip_gate_bound_cases) gate_bound_cases;
    decltype(&kt_hip_gate_portable) gate_portable;
    decltype(&kt_hip_gate_backend) gate_backend;
    decltype(&kt_hip_portable_linear) portable_linear;
    decltype(&kt_hip_equality_gate) equality_gate;
    decltype(&kt_hip_residency_gate) residency_gate;

    template <typename F>
    bool sym(F& f, const char* name) {
        f = reinterpret_cast<F>(dlsym(h, name));
        if (!f) fprintf(stderr, "kt_runtime_probe: %s lacks %s\n", name, name);
        return f != nullptr;
    }
    bool load(const std::string& path) {
        h = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
        if (!h) {
            fprintf(stderr, "kt_runtime_probe: cannot open %s: %s\n", path.c_str(), dlerror());
            return false;
        }
        return sym(device_count, "kt_hip_device_count") && sym(device_info, "kt_hip_device_info") &&
               sym(open, "kt_hip_open") && sym(open_planted, "kt_hip_open_planted") && sym(close, "kt_hip_close") &&
               sym(linear, "kt_hip_linear") && sym(linear_weights, "kt_hip_linear_weights") &&
               sym(weight_id_fresh, "kt_hip_weight_id_fresh") && sym(fallbacks, "kt_hip_fallbacks") &&
               sym(error_string, "kt_hip_error_string") && sym(gate_corpus, "kt_hip_gate_corpus") &&
               sym(gate_bound_cases, "kt_hip_gate_bound_cases") && sym(gate_portable, "kt_hip_gate_portable") &&
               sym(gate_backend, "kt_hip_gate_backend") && sym(portable_linear, "kt_hip_portable_linear") &&
               sym(equality_gate, "kt_hip_equality_gate") && sym(residency_gate, "kt_hip_residency_gate");
    }
};

std::string here() {
    char buf[PATH_MAX];
    const ssize_t n = readlink("/proc/self/exe", buf, sizeof(buf) - 1);
    if (n <= 0) return ".";
    buf[n] = 0;
    std::string p(buf);
    const size_t s = p.rfind('/');
    return s == std::string::npos ? "." : p.substr(0, s);
}

std::string diverged_labels(uint64_t mask, const kt_gate_case* cases, size_t n) {
    std::string s = "[";
    for (size_t c = 0; c < n; c++)
        if (mask >> c & 1) s += std::string(s.size() > 1 ? ", " : "") + "\"" + cases[c].label + "\"";
    return s + "]";
}

bool bound_ok(const kt_gate_backend& b, const kt_gate_case& c, const Lib& L) {
    std::vector<int64_t> got(c.rows * c.out), want(c.rows * c.out);
    if (b.linear_weights(b.ctx, c.x, c.id, c.w, c.rows, c.out, c.k, got.data())) return false;
    L.portable_linear(c.x, c.w, c.rows, c.out, c.k, want.data());
    return got == want;
}

}  // namespace

int main(int argc, char** argv) {
    bool budget1 = false, plants = false, speed = true;
    for (int i = 1; i < argc; i++) {
        if (!strcmp(argv[i], "--budget-1")) budget1 = true;
        else if (!strcmp(argv[i], "--plants")) plants = true;
        else if (!strcmp(argv[i], "--no-speed")) speed = false;
        else {
            fprintf(stderr, "usage: %s [--budget-1] [--plants] [--no-speed]\n", argv[0]);
            return 2;
        }
    }
    const std::string dir = here();
    Lib L;
    if (!L.load(dir + "/libkt_hip.so")) return 2;

    struct utsname u;
    uname(&u);
    printf("kt-runtime probe (tritify-amd)\n");
    printf("  host        : %s / %s \xc2\xb7 %u cores\n", u.machine, u.sysname, std::thread::hardware_concurrency());
    printf("  cpu variants: [\"portable\"]\n");
    int ndev = 0;
    if (L.device_count(&ndev)) ndev = 0;
    for (int d = 0; d < ndev; d++) {
        char name[256] = {0};
        int major = 0, minor = 0;
        size_t free_bytes = 0;
        L.device_info(d, name, sizeof(name), &major, &minor, &free_bytes);
        printf("  gpu %d       : hip / %s (arch %d.%d, %.1f GiB free)\n", d, name, major, minor,
               free_bytes / 1073741824.0);
    }
    if (ndev == 0) printf("  gpu         : none\n");

    std::vector<kt_gate_backend> backends(1);
    std::vector<kt_hip_backend*> opened;
    L.gate_portable(&backends[0]);
    if (ndev > 0) {
        for (uint64_t budget : budget1 ? std::vector<uint64_t>{0, 1} : std::vector<uint64_t>{0}) {
            kt_hip_backend* b = nullptr;
            const int e = L.open(0, budget, &b);
            if (e) {
                printf("  open        : device 0 failed: %s\n", L.error_string(e));
                return 1;
            }
            opened.push_back(b);
            kt_gate_backend g;
            L.gate_backend(b, &g);
            backends.push_back(g);
        }
    }
    printf("  auto        : %s\n", backends.size() > 1 ? backends[1].name : "portable");

    const kt_gate_case* cases = nullptr;
    const size_t ncases = L.gate_corpus(&cases);
    std::vector<kt_gate_report> reports(backends.size());
    const int gate = L.equality_gate(backends.data(), backends.size(), cases, ncases, reports.data());
    bool ok = gate == 0;
    if (gate != 0 && gate != KT_GATE_DIVERGED) {
        printf("  gate        : error %d\n", gate);
        return 1;
    }
    for (const auto& r : reports) {
        const std::string verdict =
            r.diverged ? "DIVERGED " + diverged_labels(r.diverged, cases, ncases) : std::string("identical");
        printf("  gate        : %-10s %s  %s\n", r.backend, r.hash, verdict.c_str());
    }
    for (size_t i = 1; i < backends.size(); i++) {
        char msg[512];
        const int e = L.residency_gate(&backends[i], cases, ncases, msg, sizeof(msg));
        ok &= e == 0;
        printf("  residency   : %-10s %s\n", backends[i].name, e == 0 ? "holds" : msg);
    }
    const kt_gate_case* bounds = nullptr;
    const size_t nb = L.gate_bound_cases(&bounds);
    for (size_t i = 1; i < backends.size(); i++)
        for (size_t c = 0; c < nb; c++) {
            const bool same = bound_ok(backends[i], bounds[c], L);
            ok &= same;
            printf("  bound       : %-10s k = %zu  %s  (%s)\n", backends[i].name, bounds[c].k,
                   same ? "identical" : "DIVERGED", bounds[c].label);
        }
    printf("  fallbacks   : %llu (calls a device backend handed to a CPU path)\n",
           (unsigned long long)L.fallbacks());

    if (plants && ndev > 0) {
        Lib P;
        if (!P.load(dir + "/libkt_hip_planted.so")) return 2;
        const struct {
            int plant;
            const char* how;
        } firing[] = {{KT_PLANT_DROP_TOP, "gate"},
                      {KT_PLANT_WRONG_CARRY, "gate"},
                      {KT_PLANT_NO_FLUSH, "bound"},
                      {KT_PLANT_CACHE_BY_SHAPE, "residency"}};
        const kt_gate_case* pc = nullptr;
        const size_t npc = P.gate_corpus(&pc);
        const kt_gate_case* pb = nullptr;
        const size_t npb = P.gate_bound_cases(&pb);
        for (const auto& f : firing) {
            kt_hip_backend* b = nullptr;
            const int e = P.open_planted(0, f.plant, &b);
            if (e) {
                printf("  plant       : %d cannot open: %s\n", f.plant, P.error_string(e));
                ok = false;
                continue;
            }
            kt_gate_backend pair[2];
            P.gate_portable(&pair[0]);
            P.gate_backend(b, &pair[1]);
            bool caught = false;
            std::string how;
            if (!strcmp(f.how, "gate")) {
                kt_gate_report r[2];
                caught = P.equality_gate(pair, 2, pc, npc, r) == KT_GATE_DIVERGED;
                how = "equality gate: diverges on " + diverged_labels(r[1].diverged, pc, npc);
            } else if (!strcmp(f.how, "bound")) {
                kt_gate_report r[2];
                const bool corpus_same = P.equality_gate(pair, 2, pc, npc, r) == 0;
                size_t caught_on = 0;
                for (size_t c = 1; c < npb; c++) caught_on += !bound_ok(pair[1], pb[c], P);
                caught = corpus_same && caught_on == npb - 1;
                how = std::string("bound cases: ") + std::to_string(caught_on) + " of " + std::to_string(npb - 1) +
                      " differ, the corpus " + (corpus_same ? "does not" : "DOES");
            } else {
                char msg[512];
                caught = P.residency_gate(&pair[1], pc, npc, msg, sizeof(msg)) == KT_GATE_DIVERGED;
                how = std::string("residency gate: ") + (caught ? msg : "holds");
            }
            ok &= caught;
            printf("  plant       : %-28s %s  %s\n", pair[1].name, caught ? "caught" : "NOT CAUGHT", how.c_str());
            P.close(b);
        }
    }

    if (speed) {  // an OLMoE-sized projection (8 rows x 2048 out x 2048 in), as runtime_probe times
        const size_t rows = 8, out = 2048, k = 2048;
        const kt_gate_case& c = cases[5];
        std::vector<int32_t> x(rows * k), w(out * k);
        for (size_t i = 0; i < x.size(); i++) x[i] = c.x[i % (c.rows * c.k)];
        for (size_t i = 0; i < w.size(); i++) w[i] = c.w[i % (c.out * c.k)];
        std::vector<int64_t> y(rows * out);
        const uint64_t id = L.weight_id_fresh();
        for (const auto& b : backends) {
            const int reps = 10;
            for (int resident = 0; resident < 2; resident++) {
                if (resident && &b == &backends[0]) continue;
                b.linear_weights(b.ctx, x.data(), resident ? id : L.weight_id_fresh(), w.data(), rows, out, k,
                                 y.data());  // warm
                const auto t0 = std::chrono::steady_clock::now();
                for (int r = 0; r < reps; r++)
                    b.linear_weights(b.ctx, x.data(), resident ? id : L.weight_id_fresh(), w.data(), rows, out, k,
                                     y.data());
                const double us =
                    std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count() / reps;
                printf("  speed       : %-10s %-16s %10.1f us/call  %8.0f MMAC/s\n", b.name,
                       resident ? "resident weights" : "fresh weights", us, rows * out * k / us);
            }
        }
    }
    for (auto* b : opened) L.close(b);
    printf("  verdict     : %s\n", ok ? "every backend byte-identical" : "A BACKEND DIVERGED");
    return ok ? 0 : 1;
}
