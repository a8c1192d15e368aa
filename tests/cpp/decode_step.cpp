// One c1 decode step through the C++ host interface (include/hip_device.hpp), in the op
// order of ziglm's GPU layer loop (cuda_model.zig:580-585, 643-662, 935-942, 953, 750):
//   addRmsNorm; rmsNormBatched(Q); rmsNormBatched(K); rope(K); kvCachePut; rope(Q);
//   geglu; tanhSoftcap.
// Usage: decode_step <in.bin> <out.bin>; the binary layouts are written/read by
// tests/test_cpp_host.py (f32 arrays in a fixed order).
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "hip_device.hpp"

using ziglm::HipBuffer;
using ziglm::HipDevice;

int main(int argc, char** argv) {
    if (argc != 3) return 2;
    const int H = 2560, nh = 8, nkv = 4, D = 256, I = 10240, pos = 1234, max_seq = 4096, S = nh * (pos + 1);
    const float eps = 1e-6f;
    const size_t sizes[] = {(size_t)H, (size_t)H, (size_t)H, (size_t)nh * D, (size_t)nkv * D, (size_t)nkv * D,
                            (size_t)D, (size_t)D, (size_t)I, (size_t)I, (size_t)S};
    std::vector<std::vector<float>> in;
    FILE* f = fopen(argv[1], "rb");
    if (!f) return 3;
    for (size_t n : sizes) {
        in.emplace_back(n);
        if (fread(in.back().data(), sizeof(float), n, f) != n) return 4;
    }
    fclose(f);
    try {
        HipDevice dev;
        std::vector<HipBuffer> d;
        for (auto& v : in) {
            d.push_back(HipBuffer::alloc(v.size() * sizeof(float)));
            d.back().upload(v.data(), v.size() * sizeof(float), dev.stream);
        }
        HipBuffer out = HipBuffer::alloc(H * sizeof(float));
        HipBuffer kc = HipBuffer::alloc((size_t)max_seq * nkv * D * sizeof(float));
        HipBuffer vc = HipBuffer::alloc((size_t)max_seq * nkv * D * sizeof(float));
        HipBuffer act = HipBuffer::alloc(I * sizeof(float));
        enum { X, R, W, Q, K, V, WQ, WK, G, U, SC };
        dev.addRmsNorm(d[X].asF32(), d[R].asConstF32(), d[W].asConstF32(), out.asF32(), H, eps, true);
        dev.rmsNormBatched(d[Q].asF32(), d[WQ].asConstF32(), d[Q].asF32(), D, nh, eps, true);
        dev.rmsNormBatched(d[K].asF32(), d[WK].asConstF32(), d[K].asF32(), D, nkv, eps, true);
        dev.rope(nullptr, d[K].asF32(), pos, 0, nkv, D, D, 10000.0f);
        dev.kvCachePut(kc.asF32(), vc.asF32(), d[K].asConstF32(), d[V].asConstF32(), 0, pos, max_seq, nkv, D, nkv * D);
        dev.rope(d[Q].asF32(), nullptr, pos, nh, 0, D, D, 10000.0f);
        dev.geglu(d[G].asConstF32(), d[U].asConstF32(), act.asF32(), I);
        dev.tanhSoftcap(d[SC].asF32(), 50.0f, S);
        dev.sync();
        if (int e = hip_bridge_last_error()) throw ziglm::HipBridgeError("op", e);
        std::vector<float> o_x(H), o_n(H), o_q(nh * D), o_k(nkv * D), o_v(nkv * D), o_a(I), o_s(S);
        d[X].download(o_x.data(), H * 4, nullptr);
        out.download(o_n.data(), H * 4, nullptr);
        d[Q].download(o_q.data(), o_q.size() * 4, nullptr);
        std::vector<float> kcache((size_t)max_seq * nkv * D), vcache((size_t)max_seq * nkv * D);
        kc.download(kcache.data(), kcache.size() * 4, nullptr);
        vc.download(vcache.data(), vcache.size() * 4, nullptr);
        act.download(o_a.data(), I * 4, nullptr);
        d[SC].download(o_s.data(), S * 4, nullptr);
        FILE* g = fopen(argv[2], "wb");
        if (!g) return 5;
        fwrite(o_x.data(), 4, H, g);
        fwrite(o_n.data(), 4, H, g);
        fwrite(o_q.data(), 4, o_q.size(), g);
        fwrite(kcache.data() + (size_t)pos * nkv * D, 4, nkv * D, g);
        fwrite(vcache.data() + (size_t)pos * nkv * D, 4, nkv * D, g);
        fwrite(o_a.data(), 4, I, g);
        fwrite(o_s.data(), 4, S, g);
        fclose(g);
        for (auto& b : d) b.deinit();
        out.deinit();
        kc.deinit();
        vc.deinit();
        act.deinit();
    } catch (const std::exception& e) {
        fprintf(stderr, "decode_step: %s\n", e.what());
        return 1;
    }
    return 0;
}
