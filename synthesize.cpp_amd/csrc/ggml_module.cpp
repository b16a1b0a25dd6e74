// The ggml dynamic-backend face of this library: libggml-hip-synth.so.
//
// synthesize.cpp finds backend modules by file name and score
// (src/backend-module.cpp:145-177): for each backend name it scans its module
// directory for libggml-<name>-*.so, dlopens each with RTLD_NOW | RTLD_LOCAL,
// calls the exported `int ggml_backend_score(void)` and keeps the highest
// non-zero score (:99-127); it then hands that file to ggml_backend_load,
// which calls the score again and then `ggml_backend_init`.
//
// This file is the half of the module that needs no ggml header:
//   - shp_module_gfx950_score: non-zero exactly when a gfx950 (MI355X) GPU is
//     visible to this process, read from the KFD topology in sysfs, which is
//     what the ROCm runtime itself enumerates. It starts no GPU runtime, so a
//     scan that dlopens and dlcloses the module stays cheap and leaves the
//     process's HIP state alone. Never throws.
//   - ggml_backend_init: the registry (reg, device, buffer and backend
//     vtables of ggml-backend-impl.h at the pinned ggml's
//     GGML_BACKEND_API_VERSION) needs those headers, absent from the
//     reference checkout; without them it returns null.
//   - ggml_backend_score: that detection only when the registry is compiled
//     in (SHP_GGML_REGISTRY, defined by a build against the pinned ggml),
//     else 0. The discovery keeps the single best-scoring libggml-hip-*.so
//     and never retries another (src/backend-module.cpp:145-177); a module
//     that outscored a working ggml HIP build and then failed in
//     ggml_backend_init would leave the process with no HIP backend. Scoring
//     0, this build loses to any real module and to the bare libggml-hip.so
//     fallback (:169-174).
//
// The node-run executor those vtables would call (graph_compute, supports_op)
// is include/synth_graph.h.
#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <dirent.h>

namespace {

constexpr unsigned long kGfx950 = 90500;  // gfx_target_version of gfx950 (9.5.0)
constexpr int           kMaxGpus = 256;

// The topology root: the kernel's, or SHP_KFD_TOPOLOGY (a copy laid out the
// same way, for tests).
const char * topology_root() {
    const char * env = std::getenv("SHP_KFD_TOPOLOGY");
    return env != nullptr && env[0] != '\0' ? env : "/sys/class/kfd/kfd/topology";
}

// gfx_target_version of topology node `node` (0: a CPU node, or unreadable).
unsigned long node_target(const char * root, long node) {
    char path[4096];
    if (std::snprintf(path, sizeof(path), "%s/nodes/%ld/properties", root, node) >= static_cast<int>(sizeof(path))) {
        return 0;
    }
    FILE * f = std::fopen(path, "r");
    if (f == nullptr) {
        return 0;
    }
    char          line[256];
    unsigned long target = 0;
    while (std::fgets(line, sizeof(line), f) != nullptr) {
        unsigned long v = 0;
        if (std::sscanf(line, "gfx_target_version %lu", &v) == 1) {
            target = v;
            break;
        }
    }
    std::fclose(f);
    return target;
}

// The GPUs of the topology in node order (what device index i of the runtime
// is before any visibility mask): their gfx_target_version values.
int gpu_targets(unsigned long (&targets)[kMaxGpus]) {
    const char * root = topology_root();
    char         path[4096];
    if (std::snprintf(path, sizeof(path), "%s/nodes", root) >= static_cast<int>(sizeof(path))) {
        return 0;
    }
    DIR * d = opendir(path);
    if (d == nullptr) {
        return 0;
    }
    long max_node = -1;
    while (const dirent * e = readdir(d)) {
        char *     end  = nullptr;
        const long node = std::strtol(e->d_name, &end, 10);
        if (end != e->d_name && *end == '\0' && node > max_node && node < 4096) {
            max_node = node;
        }
    }
    closedir(d);
    int n = 0;
    for (long node = 0; node <= max_node && n < kMaxGpus; ++node) {
        const unsigned long t = node_target(root, node);
        if (t != 0) {
            targets[n++] = t;
        }
    }
    return n;
}

// Applies a visibility list ("0,2", as ROCR_VISIBLE_DEVICES and
// HIP_VISIBLE_DEVICES take it) to targets[0..n). Entries that are not plain
// indices (UUIDs) leave the list as it is; an empty list hides every device.
int apply_visible(const char * list, unsigned long (&targets)[kMaxGpus], int n) {
    if (list == nullptr) {
        return n;
    }
    unsigned long out[kMaxGpus];
    int           m = 0;
    const char *  p = list;
    while (*p != '\0') {
        char *     end = nullptr;
        errno          = 0;
        const long i   = std::strtol(p, &end, 10);
        if (end == p || errno != 0 || (*end != ',' && *end != '\0')) {
            return n;  // not a plain index list
        }
        if (i < 0) {
            break;  // -1 and below: nothing after it is visible
        }
        if (i < n && m < kMaxGpus) {
            out[m++] = targets[i];
        }
        p = *end == ',' ? end + 1 : end;
    }
    for (int k = 0; k < m; ++k) {
        targets[k] = out[k];
    }
    return m;
}

}  // namespace

extern "C" {

// Non-zero when at least one gfx950 device is visible: 1 + the number of them
// (capped), so a module directory holding builds for several machines ranks
// this one by what it can use. 0 otherwise, including when the topology
// cannot be read. The score a registry build reports; exported under its own
// name so the detection can be checked without one.
__attribute__((visibility("default"))) int shp_module_gfx950_score(void) {
    unsigned long targets[kMaxGpus];
    int           n = gpu_targets(targets);
    n               = apply_visible(std::getenv("ROCR_VISIBLE_DEVICES"), targets, n);
    n               = apply_visible(std::getenv("HIP_VISIBLE_DEVICES"), targets, n);
    int gfx950      = 0;
    for (int k = 0; k < n; ++k) {
        gfx950 += targets[k] == kGfx950 ? 1 : 0;
    }
    return gfx950 == 0 ? 0 : 1 + (gfx950 < 64 ? gfx950 : 64);
}

// The module's score in the discovery: 0 until ggml_backend_init returns a
// registry, so that this build is never picked over one that works.
__attribute__((visibility("default"))) int ggml_backend_score(void) {
#ifdef SHP_GGML_REGISTRY
    return shp_module_gfx950_score();
#else
    return 0;
#endif
}

// The registry needs the pinned ggml's backend interface headers; this build
// has none, so there is no registry to return.
__attribute__((visibility("default"))) void * ggml_backend_init(void) {
    return nullptr;
}

}  // extern "C"
