// plan_pipeline -- the planned decode as a serving loop runs it, timed through the C ABI:
// every step the host plans the batch (kvc_decode_plan into one of a ring of pinned
// buffers) and uploads the work list on a copy stream while the GPU runs the previous
// step's kernel; the kernel waits for its upload through an event, the host waits for a
// ring slot's previous kernel before reusing the slot.
//
//   plan_pipeline <batch file> <steps> <warmup> [mode]
//
// mode 0 (default): the work list is uploaded on a copy stream; mode 1: the kernel
// reads it straight from the pinned host buffer (device-mapped host memory, one
// 64-byte entry per workgroup over PCIe), so a step costs the host one plan and one
// launch.
//
// The batch file holds int32 values: N Hq Hkv D BLOCK table_len, then lengths[N],
// tab_off[N+1], table[table_len].  K/V pools (4 copies, cycled) and q are filled with
// N(0,1) fp16 on the device.  After timing, the last step's output is compared with a
// plain planned launch on the same pool (plan made once): they must agree bit for bit.
// Prints one JSON line.
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "kvc_abi.h"

#define CK(x)                                                                        \
    do {                                                                             \
        int rc_ = (x);                                                               \
        if (rc_ != KVC_OK) {                                                         \
            std::fprintf(stderr, "%s failed: %s\n", #x, kvc_last_error());           \
            std::exit(1);                                                            \
        }                                                                            \
    } while (0)

int main(int argc, char** argv) {
    if (argc < 4) {
        std::fprintf(stderr, "usage: plan_pipeline <batch file> <steps> <warmup>\n");
        return 2;
    }
    const int steps = std::atoi(argv[2]), warmup = std::atoi(argv[3]);
    const int mode = argc > 4 ? std::atoi(argv[4]) : 0;
    std::FILE* f = std::fopen(argv[1], "rb");
    if (!f) {
        std::fprintf(stderr, "cannot open %s\n", argv[1]);
        return 2;
    }
    int hdr[6];
    if (std::fread(hdr, sizeof(int), 6, f) != 6) return 2;
    const int N = hdr[0], Hq = hdr[1], Hkv = hdr[2], D = hdr[3], B = hdr[4], table_len = hdr[5];
    std::vector<int> lens(N), tab_off(N + 1), table(table_len);
    if (std::fread(lens.data(), sizeof(int), N, f) != (size_t)N ||
        std::fread(tab_off.data(), sizeof(int), N + 1, f) != (size_t)N + 1 ||
        std::fread(table.data(), sizeof(int), table_len, f) != (size_t)table_len)
        return 2;
    std::fclose(f);
    long long tokens = 0;
    int nblocks = 0;
    for (int i = 0; i < N; ++i) tokens += lens[i];
    for (int t : table) nblocks = std::max(nblocks, t + 1);

    const int kRot = 4, kRing = 4;
    const size_t pool_elems = (size_t)nblocks * Hkv * B * D;
    void *kp[kRot], *vp[kRot], *q, *out, *out_ref, *table_d;
    for (int r = 0; r < kRot; ++r) {
        CK(kvc_malloc(&kp[r], pool_elems * 2));
        CK(kvc_malloc(&vp[r], pool_elems * 2));
        CK(kvc_fill_normal(kp[r], pool_elems, KVC_F16, 1000 + 2 * r, 1.0f, nullptr));
        CK(kvc_fill_normal(vp[r], pool_elems, KVC_F16, 1001 + 2 * r, 1.0f, nullptr));
    }
    const size_t qn = (size_t)N * Hq * D;
    CK(kvc_malloc(&q, qn * 2));
    CK(kvc_malloc(&out, qn * 2));
    CK(kvc_malloc(&out_ref, qn * 2));
    CK(kvc_fill_normal(q, qn, KVC_F16, 999, 1.0f, nullptr));
    CK(kvc_malloc(&table_d, (size_t)table_len * 4));
    CK(kvc_memcpy_h2d(table_d, table.data(), (size_t)table_len * 4, nullptr));

    const int ipu = kvc_decode_plan_entry_ints(Hq, Hkv, D, B, KVC_F16);
    int cap_units = 0;
    CK(kvc_decode_plan_capacity(N, tokens, Hq, Hkv, D, B, KVC_F16, &cap_units));
    const size_t wbytes = (size_t)cap_units * ipu * 4;
    void *host[kRing], *dev[kRing], *up_done[kRing], *k_done[kRing];
    for (int r = 0; r < kRing; ++r) {
        CK(kvc_host_alloc(&host[r], wbytes));
        CK(kvc_malloc(&dev[r], wbytes));
        CK(kvc_event_create(&up_done[r]));
        CK(kvc_event_create(&k_done[r]));
    }
    const size_t ws_bytes = std::max<size_t>(kvc_decode_planned_workspace_size(Hq, Hkv, D, B, KVC_F16, cap_units), 256);
    void* ws;
    CK(kvc_malloc(&ws, ws_bytes));
    // the fills and the table upload ran on the null stream, which the non-blocking
    // compute and copy streams do not wait for: finish them before the first step
    CK(kvc_device_synchronize());
    kvc_stream_t compute, copy;
    CK(kvc_stream_create(&compute));
    CK(kvc_stream_create(&copy));
    const float scale = 1.0f / std::sqrt((float)D);
    bool used[kRing] = {false, false, false, false};
    int nu = 0, nr = 0;

    auto step = [&](int i, void* o) {
        const int r = i % kRing;
        if (used[r]) CK(kvc_event_synchronize(k_done[r]));
        CK(kvc_decode_plan(lens.data(), tab_off.data(), table.data(), table_len, N, Hq, Hkv, D, B, KVC_F16, 0,
                           static_cast<int*>(host[r]), cap_units, &nu, &nr));
        void* wl = host[r];
        if (mode == 0) {
            CK(kvc_memcpy_h2d(dev[r], host[r], (size_t)nu * ipu * 4, copy));
            CK(kvc_event_record(up_done[r], copy));
            CK(kvc_stream_wait_event(compute, up_done[r]));
            wl = dev[r];
        }
        CK(kvc_batched_paged_decode_planned(q, kp[i % kRot], vp[i % kRot], static_cast<int*>(table_d), table_len, o,
                                            N, Hq, Hkv, D, B, scale, KVC_F16, static_cast<int*>(wl), nu, nr,
                                            ws, ws_bytes, compute));
        CK(kvc_event_record(k_done[r], compute));
        used[r] = true;
    };

    for (int i = 0; i < warmup; ++i) step(i, out);
    CK(kvc_device_synchronize());
    void *e0, *e1;
    CK(kvc_event_create(&e0));
    CK(kvc_event_create(&e1));
    CK(kvc_event_record(e0, compute));
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < steps; ++i) step(warmup + i, out);
    const double host_us =
        std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count() / steps;
    CK(kvc_event_record(e1, compute));
    float ms = 0.f;
    CK(kvc_event_elapsed_ms(&ms, e0, e1));
    CK(kvc_device_synchronize());

    // the last step's output against a plain planned launch on the same pool copy
    const int last = warmup + steps - 1;
    std::vector<int> work((size_t)cap_units * ipu);
    int nu2 = 0, nr2 = 0;
    CK(kvc_decode_plan(lens.data(), tab_off.data(), table.data(), table_len, N, Hq, Hkv, D, B, KVC_F16, 0,
                       work.data(), cap_units, &nu2, &nr2));
    CK(kvc_memcpy_h2d(dev[0], work.data(), (size_t)nu2 * ipu * 4, nullptr));
    CK(kvc_batched_paged_decode_planned(q, kp[last % kRot], vp[last % kRot], static_cast<int*>(table_d), table_len,
                                        out_ref, N, Hq, Hkv, D, B, scale, KVC_F16, static_cast<int*>(dev[0]), nu2,
                                        nr2, ws, ws_bytes, nullptr));
    CK(kvc_device_synchronize());
    std::vector<unsigned short> a(qn), b(qn);
    CK(kvc_memcpy_d2h(a.data(), out, qn * 2, nullptr));
    CK(kvc_memcpy_d2h(b.data(), out_ref, qn * 2, nullptr));
    CK(kvc_device_synchronize());
    const bool same = std::memcmp(a.data(), b.data(), qn * 2) == 0;

    std::printf("{\"mode\": \"%s\", \"us_per_step\": %.3f, \"host_us_per_step\": %.2f, \"units\": %d, \"upload_bytes_per_step\": %zu, "
                "\"steps\": %d, \"output_equals_plain_planned_launch\": %s}\n",
                mode == 0 ? "work list uploaded on a copy stream" : "kernel reads the work list from pinned host memory",
                ms * 1000.0 / steps, host_us, nu, (size_t)nu * ipu * 4, steps, same ? "true" : "false");
    for (int r = 0; r < kRing; ++r) {
        kvc_host_free(host[r]);
        kvc_free(dev[r]);
        kvc_event_destroy(up_done[r]);
        kvc_event_destroy(k_done[r]);
    }
    for (int r = 0; r < kRot; ++r) {
        kvc_free(kp[r]);
        kvc_free(vp[r]);
    }
    kvc_free(q);
    kvc_free(out);
    kvc_free(out_ref);
    kvc_free(table_d);
    kvc_free(ws);
    kvc_event_destroy(e0);
    kvc_event_destroy(e1);
    kvc_stream_destroy(compute);
    kvc_stream_destroy(copy);
    return same ? 0 : 1;
}
