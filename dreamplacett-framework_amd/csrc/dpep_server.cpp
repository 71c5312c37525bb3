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
// density, the potential and the per-cell forces.
//
// Environment honoured as in the reference: EXPORT_DENSITY_PATH (density
// every step, float[M*N]), EXPORT_POS_PATH (positions at steps 1, 50, 100,
// :1686-1726 format), CPU_DCT=1 (density in the field_x slot, field_y zero,
// :1785-1788), GATHER_MODE (accepted, no effect).
#include <fcntl.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <chrono>
#include <string>
#include <vector>

#include "dpep.h"

namespace {

constexpr uint32_t kIdle = 0, kGo = 1, kDone = 2, kQuit = 3;
constexpr size_t kHeader = 64;
constexpr uint32_t kMagicV2 = 0x32504544u;
constexpr uint32_t kOutDensity = 1u, kOutPotential = 2u, kOutGrads = 4u;
constexpr uint32_t kGatherModeHip = 16u;

double now_ms()
{
    using namespace std::chrono;
    return duration<double, std::milli>(steady_clock::now().time_since_epoch()).count();
}

void flag_write(const std::string& path, const char* content)
{
    const std::string tmp = path + ".tmp";
    FILE* f = fopen(tmp.c_str(), "w");
    if (!f) {
        perror(("fopen " + tmp).c_str());
        return;
    }
    fputs(content, f);
    fclose(f);
    rename(tmp.c_str(), path.c_str());
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

    dpep_ctx* ctx = nullptr;
    // the shm header reports every step's timings
    if (dpep_create(M, N, NC_max, xl, yl, xh, yh, DPEP_DTYPE_F32, DPEP_FLAG_STEP_TIMINGS,
                    &ctx) != DPEP_OK)
        fatal("dpep_create");

    // Open the shm file the client created (poll briefly, :1258-1267).
    int fd = -1;
    for (int i = 0; i < 100 && fd < 0; ++i) {
        fd = open(shm_path.c_str(), O_RDWR);
        if (fd < 0) usleep(100000);
    }
    if (fd < 0) {
        perror(("[server] open shm: " + shm_path).c_str());
        return 1;
    }
    struct stat st;
    if (fstat(fd, &st) != 0) {
        perror("[server] fstat shm");
        return 1;
    }
    const size_t soa = ((size_t)NC_max + 1023) / 1024 * 1024;
    const size_t pos_bytes = soa * 4, map_bytes = (size_t)M * N * 4;
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
        perror("[server] mmap shm");
        return 1;
    }
    char* p = (char*)base;
    volatile uint32_t* state = (volatile uint32_t*)p;
    volatile int32_t* shm_nc = (volatile int32_t*)(p + 4);
    float* timing = (float*)(p + 8);
    uint32_t* gmode = (uint32_t*)(p + 44);
    const uint32_t* hdr_v2 = (const uint32_t*)(p + 48);
    const float* px = (const float*)(p + kHeader);
    const float* py = px + soa;
    const float* sx = py + soa;
    const float* sy = sx + soa;
    float* fx = (float*)(p + kHeader + 4 * pos_bytes);
    float* fy = fx + (size_t)M * N;
    const float* init_density = fy + (size_t)M * N;
    float* density = nullptr;
    float* potential = nullptr;
    float* gx = nullptr;
    float* gy = nullptr;
    if (hdr_v2[0] == kMagicV2 && shm_size >= v2_size) {
        float* d = (float*)(p + v1_size);
        density = d;
        potential = d + (size_t)M * N;
        gx = (float*)(p + v1_size + 2 * map_bytes);
        gy = gx + soa;
        printf("[server] shm version 2 (density, potential, per-cell forces)\n");
    } else {
        printf("[server] shm version 1 (fields only)\n");
    }
    fflush(stdout);

    flag_write(ready_flag, "READY\n");
    printf("[server] READY -- polling shm state\n");
    fflush(stdout);

    std::vector<float> dens_host;       // density for CPU_DCT / export
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
            if (dpep_set_initial_density(ctx, init_density) != DPEP_OK)
                fatal("dpep_set_initial_density");
            d0_uploaded = true;
        }
        const uint32_t outs = density ? hdr_v2[2] : 0u;
        const char* dump_dens = getenv("EXPORT_DENSITY_PATH");
        const bool want_dens_host = cpu_dct || (dump_dens && dump_dens[0]);
        float* dens_out = (outs & kOutDensity) ? density : nullptr;
        if (want_dens_host && !dens_out) {
            dens_host.resize((size_t)M * N);
            dens_out = dens_host.data();
        }
        const double tf0 = now_ms();
        int rc;
        if (cpu_dct) {
            rc = dpep_step(ctx, px, py, sx, sy, nc, nullptr, nullptr, dens_out, nullptr,
                           nullptr, nullptr);
        } else {
            rc = dpep_step(ctx, px, py, sx, sy, nc, fx, fy, dens_out,
                           (outs & kOutPotential) ? potential : nullptr,
                           (outs & kOutGrads) ? gx : nullptr,
                           (outs & kOutGrads) ? gy : nullptr);
        }
        if (rc != DPEP_OK) fatal("dpep_step");
        float t[DPEP_NUM_TIMINGS] = {0};
        dpep_get_timings(ctx, t);
        const double tw0 = now_ms();
        if (cpu_dct) {
            memcpy(fx, dens_out, map_bytes);
            memset(fy, 0, map_bytes);
        }
        if (dump_dens && dump_dens[0]) {
            FILE* f = fopen(dump_dens, "wb");
            if (f) {
                fwrite(dens_out, 4, (size_t)M * N, f);
                fclose(f);
            }
        }
        const char* dump_pos = getenv("EXPORT_POS_PATH");
        if (dump_pos && dump_pos[0] && (iter == 1 || iter == 50 || iter == 100))
            dump_positions(dump_pos, iter, M, N, xl, yl, xh, yh, nc, px, py, sx, sy);
        const double t1 = now_ms();
        (void)tf0;
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
        printf("[server] done nc=%d h2d=%.3f compute=%.3f download=%.3f total=%.3f\n", nc,
               t[0], t[5], t[6], t1 - t0);
        fflush(stdout);
    }
    munmap(base, shm_size);
    dpep_destroy(ctx);
    return 0;
}
