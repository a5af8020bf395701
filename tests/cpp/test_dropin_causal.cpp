// test_dropin_causal.cpp -- the drop-in qkcuda_paged_causal_attn (include/kvc/qwen_kernels.h,
// the reference's qwen_kernels.h:45-47) outside and under stream capture.
//   * Outside capture it takes the library's per-stream workspace, so a prompt of 40
//     queries (past the allocation-free entry point's static scratch) runs and equals
//     kvc_paged_causal_attn_dev with a caller workspace bit for bit (same kernel, same plan).
//   * Under capture it takes the allocation-free entry point: one query per step, as the
//     reference captures it (qwen_infer.cu:145-162), replays equal eager launches bit for bit
//     over three replays with eager work between them; a 40-query call under capture is
//     refused with KVC_ERR_UNSUPPORTED before anything is recorded.
#include <cstdio>
#include <cstring>
#include <vector>

#include "kvc/qwen_kernels.h"

#define OK(x) do { int rc_ = (x); if (rc_) { std::printf("FAIL %s: %s\n", #x, kvc_last_error()); return 2; } } while (0)
#define EXPECT(c) do { if (!(c)) { std::printf("FAIL %s\n", #c); return 1; } } while (0)

static bool same(void* a, void* b, size_t bytes) {
    std::vector<unsigned char> x(bytes), y(bytes);
    if (kvc_memcpy_d2h(x.data(), a, bytes, nullptr) || kvc_memcpy_d2h(y.data(), b, bytes, nullptr)) return false;
    return std::memcmp(x.data(), y.data(), bytes) == 0;
}

int main() {
    const int Hq = 14, Hkv = 2, D = 64, B = 16, base = 1000, NqBig = 40;
    const float scale = 0.125f;
    const int nb = (base + NqBig + B - 1) / B + 3;
    std::vector<int> table(nb);
    for (int i = 0; i < nb; ++i) table[i] = (i * 7) % nb;  // a permutation (7 and nb coprime)
    if (nb % 7 == 0) return 3;
    const size_t pool = (size_t)nb * Hkv * B * D, qn = (size_t)NqBig * Hq * D;
    void *kp, *vp, *q, *o1, *o2, *dt, *pos, *ws;
    OK(kvc_malloc(&kp, pool * 2)); OK(kvc_malloc(&vp, pool * 2)); OK(kvc_malloc(&q, qn * 2));
    OK(kvc_malloc(&o1, qn * 2)); OK(kvc_malloc(&o2, qn * 2)); OK(kvc_malloc(&dt, nb * 4)); OK(kvc_malloc(&pos, 4));
    OK(kvc_fill_normal(kp, pool, KVC_F16, 11, 1.0f, nullptr));
    OK(kvc_fill_normal(vp, pool, KVC_F16, 12, 1.0f, nullptr));
    OK(kvc_fill_normal(q, qn, KVC_F16, 13, 1.0f, nullptr));
    OK(kvc_memcpy_h2d(dt, table.data(), nb * 4, nullptr));
    OK(kvc_memcpy_h2d(pos, &base, 4, nullptr));
    const size_t wsb = kvc_paged_causal_attn_dev_workspace_size(NqBig, Hq, Hkv, D, B, KVC_F16);
    EXPECT(wsb > 0);
    OK(kvc_malloc(&ws, wsb));
    OK(kvc_device_synchronize());
    kvc_stream_t st;
    OK(kvc_stream_create(&st));
    half *hq = (half*)q, *h1 = (half*)o1, *h2 = (half*)o2, *hk = (half*)kp, *hv = (half*)vp;

    // outside capture: 40 queries through the drop-in
    OK(qkcuda_paged_causal_attn(hq, h1, hk, hv, (const int*)dt, (int*)pos, NqBig, Hq, Hkv, D, B, scale, st));
    OK(kvc_paged_causal_attn_dev(q, o2, kp, vp, (const int*)dt, (const int*)pos, NqBig, Hq, Hkv, D, B, scale, KVC_F16,
                                 ws, wsb, st));
    OK(kvc_stream_synchronize(st));
    EXPECT(same(o1, o2, qn * 2));
    std::printf("eager 40 queries: drop-in equals the workspace entry point\n");

    // under capture: one query per step
    int capturing = 0;
    OK(kvc_stream_is_capturing(st, &capturing));
    EXPECT(capturing == 0);
    OK(kvc_graph_begin(st));
    OK(kvc_stream_is_capturing(st, &capturing));
    EXPECT(capturing == 1);
    OK(qkcuda_paged_causal_attn(hq, h1, hk, hv, (const int*)dt, (int*)pos, 1, Hq, Hkv, D, B, scale, st));
    void* exec = nullptr;
    OK(kvc_graph_end(st, &exec));
    const size_t one = (size_t)Hq * D * 2;
    for (int r = 0; r < 3; ++r) {
        const int p = base + 5 * r;
        OK(kvc_memcpy_h2d(pos, &p, 4, st));
        OK(kvc_memset(o1, 0, one, st));
        OK(kvc_graph_launch(exec, st));
        OK(kvc_paged_causal_attn_dev(q, o2, kp, vp, (const int*)dt, (const int*)pos, 1, Hq, Hkv, D, B, scale, KVC_F16,
                                     ws, wsb, st));
        OK(kvc_stream_synchronize(st));
        EXPECT(same(o1, o2, one));
    }
    OK(kvc_graph_destroy(exec));
    std::printf("captured one-query step: three replays equal eager launches\n");

    // under capture, a call past the static scratch is refused
    OK(kvc_graph_begin(st));
    const int rc = qkcuda_paged_causal_attn(hq, h1, hk, hv, (const int*)dt, (int*)pos, NqBig, Hq, Hkv, D, B, scale, st);
    void* exec2 = nullptr;
    const int rc_end = kvc_graph_end(st, &exec2);
    if (exec2) OK(kvc_graph_destroy(exec2));
    EXPECT(rc == KVC_ERR_UNSUPPORTED);
    EXPECT(rc_end == KVC_OK);
    std::printf("captured 40-query call refused: %s\n", "KVC_ERR_UNSUPPORTED");

    OK(kvc_stream_destroy(st));
    for (void* p : {kp, vp, q, o1, o2, dt, pos, ws}) OK(kvc_free(p));
    std::printf("PASS\n");
    return 0;
}
