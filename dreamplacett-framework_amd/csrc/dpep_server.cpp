// dpep_server.cpp -- density_scatter_hip_server: the shared-memory server of
// the electric-potential step, a drop-in for the reference's
// density_scatter_ttnn_server (host/density_scatter_ttnn_server_host.cpp).
//
//   density_scatter_hip_server M N NC_max ipc_dir [xl yl xh yh]
//
// Same command line (:324-339), same ready.flag written by tmp + rename after
// start-up (:312-318, :1293), same shm state machine (:1326-1824): poll the
// state word, on GO run one step on nc = min(nc_actual, NC_max) cells, write
// the fields and the 9 timing slots, set DONE; QUIT ends the server.  The
// device work goes through libdpep.so's C ABI (include/dpep.h).  Version-2
// shm files (magic in the header padding, see dpep/shm.py) also receive the
// density, the potential and the per-cell forces, as the header's output
// word asks, and may ask for no fields at all.
//
// Transfers: the positions are copied from the shm file into page-locked
// staging buffers (dpep_host_alloc) by a few threads, uploaded from there,
// and the requested outputs come back the same way; only the slots a step
// needs cross the link.
//
// Environment honoured as in the reference: EXPORT_DENSITY_PATH (the
// scattered cells' density every step, float[M*N], before the initial
// density is added, :1676-1695), EXPORT_POS_PATH (positions at steps 1, 50,
// 100, :1696-1726 format), CPU_DCT=1 (that same density, without the
// initial density, in the field_x slot and field_y zero, :1757-1788; the
// client adds the initial density back and solves on the CPU), GATHER_MODE
// (accepted, no effect).
#include <errno.h>
#include <fcntl.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <string>
#include <thread>
#include <vector>

#include "dpep.h"
#include "dpep_copy_pool.h"

namespace {

constexpr uint32_t kIdle = 0, kGo = 1, kDone = 2, kQuit = 3;
constexpr size_t kHeader = 64;
constexpr uint32_t kMagicV2 = 0x32504544u;
constexpr uint32_t kOutDensity = 1u, kOutPotential = 2u, kOutGrads = 4u, kOutNoFields = 8u;
// input bit of the same word: the client did not rewrite the size slots
constexpr uint32_t kInKeepSizes = 0x10u;
constexpr uint32_t kGatherModeHip = 16u;

double now_ms()
{
    using namespace std::chrono;
    return duration<double, std::milli>(steady_clock::now().time_since_epoch()).count();
}

// Publishes `content` at `path` atomically: written to a sibling file first,
// then renamed over the target, so a poller never reads a partial flag.
void publish_flag(const std::string& path, const char* content)
{
    const std::string part = path + ".tmp";
    FILE* f = fopen(part.c_str(), "w");
    if (!f) {
        fprintf(stderr, "[server] cannot write %s\n", part.c_str());
        return;
    }
    fputs(content, f);
    fclose(f);
    if (rename(part.c_str(), path.c_str()) != 0)
        fprintf(stderr, "[server] cannot rename %s\n", part.c_str());
}

float* host_floats(size_t n)
{
    void* p = nullptr;
    if (dpep_host_alloc(n * sizeof(float), &p) != DPEP_OK) return nullptr;
    return (float*)p;
}

[[noreturn]] void fatal(const char* what)
{
    fprintf(stderr, "[server] FATAL %s: %s\n", what, dpep_last_error());
    fflush(stderr);
    exit(1);
}

void dump_positions(const char* base, uint32_t iter, int M, int N, float xl,
                    float yl, float xh, float yh, int32_t nc, const float* px,
                    const float* py, const float* sx, const float* sy)
{
    char path[1024];
    snprintf(path, sizeof path, "%s.iter%u.bin", base, iter);
    FILE* f = fopen(path, "wb");
    if (!f) return;
    int32_t Mi = M, Ni = N;
    fwrite(&Mi, 4, 1, f);
    fwrite(&Ni, 4, 1, f);
    fwrite(&xl, 4, 1, f);
    fwrite(&yl, 4, 1, f);
    fwrite(&xh, 4, 1, f);
    fwrite(&yh, 4, 1, f);
    fwrite(&nc, 4, 1, f);
    fwrite(px, 4, (size_t)nc, f);
    fwrite(py, 4, (size_t)nc, f);
    fwrite(sx, 4, (size_t)nc, f);
    fwrite(sy, 4, (size_t)nc, f);
    fclose(f);
}

}  // namespace

int main(int argc, char** argv)
{
    if (argc < 5) {
        fprintf(stderr, "Usage: %s M N NC_max ipc_dir [xl yl xh yh]\n", argv[0]);
        return 1;
    }
    const int M = atoi(argv[1]);
    const int N = atoi(argv[2]);
    const int NC_max = atoi(argv[3]);
    const std::string ipc_dir = argv[4];
    float xl = 0.f, yl = 0.f, xh = 1e6f, yh = 1e6f;
    if (argc >= 9) {
        xl = (float)atof(argv[5]);
        yl = (float)atof(argv[6]);
        xh = (float)atof(argv[7]);
        yh = (float)atof(argv[8]);
    }
    const std::string shm_path = ipc_dir + "/scatter.shm";
    const std::string ready_flag = ipc_dir + "/ready.flag";
    const char* cpu_dct_env = getenv("CPU_DCT");
    const bool cpu_dct = cpu_dct_env && std::string(cpu_dct_env) == "1";
    printf("[server] M=%d N=%d NC_max=%d die=[%g,%g]x[%g,%g] (%s)\n", M, N, NC_max,
           xl, xh, yl, yh, dpep_build_info());
    fflush(stdout);

    const char* dump_dens = getenv("EXPORT_DENSITY_PATH");
    const bool dump_density = dump_dens && dump_dens[0];
    const char* dump_pos = getenv("EXPORT_POS_PATH");

    // the shm header reports every step's timings; the reference's dump and
    // CPU-solve mode need the scattered cells' density before the fold
    unsigned flags = DPEP_FLAG_STEP_TIMINGS;
    if (cpu_dct || dump_density) flags |= DPEP_FLAG_SCATTER_DENSITY;
    dpep_ctx* ctx = nullptr;
    if (dpep_create(M, N, NC_max, xl, yl, xh, yh, DPEP_DTYPE_F32, flags, &ctx) != DPEP_OK)
        fatal("dpep_create");

    // The client creates the shm file before it launches the server; allow
    // it up to ten seconds to appear (:1258-1267 polls the same way).
    int fd = -1;
    const double open_deadline = now_ms() + 10000.0;
    while ((fd = open(shm_path.c_str(), O_RDWR)) < 0 && now_ms() < open_deadline)
        usleep(50000);
    if (fd < 0) {
        fprintf(stderr, "[server] FATAL cannot open %s: %s\n", shm_path.c_str(),
                strerror(errno));
        return 1;
    }
    struct stat st;
    if (fstat(fd, &st) != 0) {
        fprintf(stderr, "[server] FATAL fstat %s: %s\n", shm_path.c_str(), strerror(errno));
        return 1;
    }
    const size_t soa = ((size_t)NC_max + 1023) / 1024 * 1024;
    const size_t MN = (size_t)M * N;
    const size_t pos_bytes = soa * 4, map_bytes = MN * 4;
    const size_t v1_size = kHeader + 4 * pos_bytes + 3 * map_bytes;
    const size_t v2_size = v1_size + 2 * map_bytes + 2 * pos_bytes;
    if ((size_t)st.st_size < v1_size) {
        fprintf(stderr, "[server] FATAL shm is %lld bytes, need %zu for M=%d N=%d NC_max=%d\n",
                (long long)st.st_size, v1_size, M, N, NC_max);
        return 1;
    }
    const size_t shm_size = (size_t)st.st_size;
    void* base = mmap(nullptr, shm_size, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
    close(fd);
    if (base == MAP_FAILED) {
        fprintf(stderr, "[server] FATAL mmap %s: %s\n", shm_path.c_str(), strerror(errno));
        return 1;
    }
    char* p = (char*)base;
    volatile uint32_t* state = (volatile uint32_t*)p;
    volatile int32_t* shm_nc = (volatile int32_t*)(p + 4);
    float* timing = (float*)(p + 8);
    uint32_t* gmode = (uint32_t*)(p + 44);
    const volatile uint32_t* hdr_v2 = (const volatile uint32_t*)(p + 48);
    const float* shm_px = (const float*)(p + kHeader);
    const float* shm_py = shm_px + soa;
    const float* shm_sx = shm_py + soa;
    const float* shm_sy = shm_sx + soa;
    float* shm_fx = (float*)(p + kHeader + 4 * pos_bytes);
    float* shm_fy = shm_fx + MN;
    const float* shm_d0 = shm_fy + MN;
    float* shm_density = nullptr;
    float* shm_potential = nullptr;
    float* shm_gx = nullptr;
    float* shm_gy = nullptr;
    const bool v2 = hdr_v2[0] == kMagicV2 && shm_size >= v2_size;
    if (v2) {
        shm_density = (float*)(p + v1_size);
        shm_potential = shm_density + MN;
        shm_gx = (float*)(p + v1_size + 2 * map_bytes);
        shm_gy = shm_gx + soa;
        printf("[server] shm version 2 (density, potential, per-cell forces)\n");
    } else {
        printf("[server] shm version 1 (fields only)\n");
    }
    fflush(stdout);

    // page-locked staging: cells in, every output a step can ask for out
    float* h_cells = host_floats(4 * soa);
    float* h_fx = host_floats(MN);
    float* h_fy = host_floats(MN);
    float* h_raw = (flags & DPEP_FLAG_SCATTER_DENSITY) ? host_floats(MN) : nullptr;
    float* h_dens = v2 ? host_floats(MN) : nullptr;
    float* h_phi = v2 ? host_floats(MN) : nullptr;
    float* h_g = v2 ? host_floats(2 * soa) : nullptr;
    if (!h_cells || !h_fx || !h_fy || ((flags & DPEP_FLAG_SCATTER_DENSITY) && !h_raw) ||
        (v2 && (!h_dens || !h_phi || !h_g)))
        fatal("dpep_host_alloc");
    float* h_px = h_cells;
    float* h_py = h_px + soa;
    float* h_sx = h_py + soa;
    float* h_sy = h_sx + soa;
    const unsigned hw = std::thread::hardware_concurrency();
    dpep::CopyPool pool((int)std::min(7u, hw > 1 ? hw - 1 : 1u));

    publish_flag(ready_flag, "READY\n");
    printf("[server] READY -- polling shm state\n");
    fflush(stdout);

    bool d0_uploaded = false;
    uint32_t iter = 0;
    while (true) {
        const uint32_t s = *state;
        if (s == kQuit) {
            printf("[server] QUIT received.\n");
            fflush(stdout);
            break;
        }
        if (s != kGo) {
            usleep(500);
            continue;
        }
        __atomic_thread_fence(__ATOMIC_ACQUIRE);
        int32_t nc = *shm_nc;
        if (nc < 0) nc = 0;
        if (nc > NC_max) nc = NC_max;
        ++iter;
        const double t0 = now_ms();
        if (!d0_uploaded) {
            // the client writes slot 3 once before its first GO (:1770-1773)
            if (dpep_set_initial_density(ctx, shm_d0) != DPEP_OK)
                fatal("dpep_set_initial_density");
            d0_uploaded = true;
        }
        // outputs this step: the fields (v1 always; v2 unless the client
        // opts out, and never in the CPU-solve mode, where the fx slot
        // carries the density), and the v2 extras the header asks for
        const uint32_t outs = v2 ? hdr_v2[2] : 0u;
        const bool want_fields = !cpu_dct && !(outs & kOutNoFields);
        const bool want_dens = (outs & kOutDensity) != 0;
        const bool want_phi = (outs & kOutPotential) != 0;
        const bool want_grads = (outs & kOutGrads) != 0;
        const size_t ncb = (size_t)nc * sizeof(float);
        const bool keep_sizes = (outs & kInKeepSizes) != 0;
        if (keep_sizes)
            pool.copy({{h_px, shm_px, ncb}, {h_py, shm_py, ncb}});
        else
            pool.copy({{h_px, shm_px, ncb}, {h_py, shm_py, ncb}, {h_sx, shm_sx, ncb},
                       {h_sy, shm_sy, ncb}});
        if (dpep_set_cells(ctx, h_px, h_py, keep_sizes ? nullptr : h_sx,
                           keep_sizes ? nullptr : h_sy, nc) != DPEP_OK)
            fatal("dpep_set_cells");
        if (dpep_compute(ctx) != DPEP_OK) fatal("dpep_compute");
        if (dpep_get_outputs(ctx, want_dens ? h_dens : nullptr, want_phi ? h_phi : nullptr,
                             want_fields ? h_fx : nullptr, want_fields ? h_fy : nullptr,
                             want_grads ? h_g : nullptr, want_grads ? h_g + soa : nullptr) !=
            DPEP_OK)
            fatal("dpep_get_outputs");
        if (h_raw && dpep_get_scatter_density(ctx, h_raw) != DPEP_OK)
            fatal("dpep_get_scatter_density");
        float t[DPEP_NUM_TIMINGS] = {0};
        dpep_get_timings(ctx, t);
        const double tw0 = now_ms();
        std::vector<dpep::CopyPool::Job> out;
        if (cpu_dct) {
            out.push_back({shm_fx, h_raw, map_bytes});
            memset(shm_fy, 0, map_bytes);
        } else if (want_fields) {
            out.push_back({shm_fx, h_fx, map_bytes});
            out.push_back({shm_fy, h_fy, map_bytes});
        }
        if (want_dens) out.push_back({shm_density, h_dens, map_bytes});
        if (want_phi) out.push_back({shm_potential, h_phi, map_bytes});
        if (want_grads) {
            out.push_back({shm_gx, h_g, ncb});
            out.push_back({shm_gy, h_g + soa, ncb});
        }
        pool.copy(out);
        if (dump_density) {
            FILE* f = fopen(dump_dens, "wb");
            if (f) {
                fwrite(h_raw, sizeof(float), MN, f);
                fclose(f);
            }
        }
        if (dump_pos && dump_pos[0] && (iter == 1 || iter == 50 || iter == 100))
            dump_positions(dump_pos, iter, M, N, xl, yl, xh, yh, nc, h_px, h_py, h_sx, h_sy);
        const double t1 = now_ms();
        timing[0] = t[0];                      // h2d
        timing[1] = t[1];                      // scatter
        timing[2] = t[2];                      // gather
        timing[3] = t[3];                      // d2h density
        timing[4] = 0.f;                       // upload (no per-step upload)
        timing[5] = t[5];                      // compute
        timing[6] = t[6];                      // download
        timing[7] = (float)(t1 - tw0);         // field write / dumps
        timing[8] = (float)(t1 - t0);          // total
        *gmode = kGatherModeHip;
        __atomic_thread_fence(__ATOMIC_RELEASE);
        *state = kDone;
        printf("[server] done nc=%d h2d=%.3f compute=%.3f download=%.3f fw=%.3f total=%.3f\n",
               nc, t[0], t[5], t[6], t1 - tw0, t1 - t0);
        fflush(stdout);
    }
    munmap(base, shm_size);
    dpep_destroy(ctx);
    for (float* h : {h_cells, h_fx, h_fy, h_raw, h_dens, h_phi, h_g}) dpep_host_free(h);
    return 0;
}
