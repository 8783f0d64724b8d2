// Exercises the C++ drop-in headers (FlashAttention.h / OlmoAttention.h mirrors)
// the way the reference's callers use them.
//
//   dropin_check cpu                       argument errors throw, no GPU needed
//   dropin_check flash <dir> B T H         reads q/k/v.f32 from dir, writes o/m/l.f32
//   dropin_check bwd <dir> B T H           reads g/o/q/k/v.f32 and m/l.f32, writes dq/dk/dv.f32
//   dropin_check layer <folder> <idx> <dir> B T   reads x.f32 and g.f32, writes out.f32 and dx.f32
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <iostream>
#include <string>

#include "dirktensor_amd/FlashAttention.h"
#include "dirktensor_amd/OlmoAttention.h"

template <class Tn>
static void read_raw(const std::string& path, Tn& t) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open " + path);
    f.read(reinterpret_cast<char*>(t.data()), (std::streamsize)(t.size() * sizeof(float)));
    if (!f) throw std::runtime_error("short read " + path);
}

template <class Tn>
static void write_raw(const std::string& path, const Tn& t) {
    std::ofstream f(path, std::ios::binary);
    f.write(reinterpret_cast<const char*>(t.data()), (std::streamsize)(t.size() * sizeof(float)));
}

template <class F>
static bool throws(F&& f) {
    try {
        f();
    } catch (const std::runtime_error& e) {
        std::cout << "  threw: " << e.what() << "\n";
        return true;
    }
    return false;
}

int main(int argc, char** argv) {
    if (argc < 2) return 2;
    const std::string mode = argv[1];
    const float scale = 1.0f / std::sqrt(128.0f);
    if (mode == "cpu") {
        auto a = dt::tensor<float, 4>::from_shape({1, 8, 2, 128});
        auto b = dt::tensor<float, 4>::from_shape({1, 9, 2, 128});
        auto c = dt::tensor<float, 4>::from_shape({1, 8, 2, 64});
        auto big = dt::tensor<float, 4>::from_shape({1, 8193, 1, 128});
        auto m3 = dt::tensor<float, 3>::from_shape({1, 8, 2});
        bool ok = true;
        ok &= throws([&] { flash_attention_forward(a, b, a, scale); });
        ok &= throws([&] { flash_attention_forward(c, c, c, scale); });
        ok &= throws([&] { flash_attention_forward(big, big, big, scale, true); });
        ok &= throws([&] { flash_attention_backward(a, b, m3, m3, a, a, a, scale); });
        ok &= throws([&] { flash_attention_backward(c, c, m3, m3, c, c, c, scale); });
        ok &= throws([&] { OlmoAttention("/nonexistent-folder", 0); });
        a(0, 3, 1, 5) = 2.5f;
        ok &= a.data()[(3 * 2 + 1) * 128 + 5] == 2.5f;
        std::cout << (ok ? "OK" : "FAIL") << "\n";
        return ok ? 0 : 1;
    }
    if (mode == "flash" && argc == 6) {
        const std::string dir = argv[2];
        const size_t B = std::atoi(argv[3]), T = std::atoi(argv[4]), H = std::atoi(argv[5]);
        auto Q = dt::tensor<float, 4>::from_shape({B, T, H, 128});
        auto K = Q, V = Q;
        read_raw(dir + "/q.f32", Q);
        read_raw(dir + "/k.f32", K);
        read_raw(dir + "/v.f32", V);
        FlashAttentionResult r = flash_attention_forward(Q, K, V, scale);
        write_raw(dir + "/o.f32", r.output);
        write_raw(dir + "/m.f32", r.softmax_m);
        write_raw(dir + "/l.f32", r.softmax_l);
        std::cout << "OK\n";
        return 0;
    }
    if (mode == "layer" && argc == 7) {
        const std::string folder = argv[2], dir = argv[4];
        const unsigned idx = (unsigned)std::atoi(argv[3]);
        const size_t B = std::atoi(argv[5]), T = std::atoi(argv[6]);
        OlmoAttention attn(folder, idx);
        auto x = dt::tensor<float, 3>::from_shape({B, T, 2048});
        read_raw(dir + "/x.f32", x);
        auto out = attn.forward(x);
        write_raw(dir + "/out.f32", out);
        auto g = x;
        read_raw(dir + "/g.f32", g);
        attn.zero_grad();
        auto dx = attn.backward(g);
        write_raw(dir + "/dx.f32", dx);
        bool ok = throws([&] { attn.backward(dt::tensor<float, 3>::from_shape({B, T + 1, 2048})); });
        std::cout << (ok ? "OK" : "FAIL") << "\n";
        return ok ? 0 : 1;
    }
    if (mode == "bwd" && argc == 6) {
        const std::string dir = argv[2];
        const size_t B = std::atoi(argv[3]), T = std::atoi(argv[4]), H = std::atoi(argv[5]);
        auto G = dt::tensor<float, 4>::from_shape({B, T, H, 128});
        auto O = G, Q = G, K = G, V = G;
        auto m = dt::tensor<float, 3>::from_shape({B, T, H});
        auto l = m;
        read_raw(dir + "/g.f32", G);
        read_raw(dir + "/o.f32", O);
        read_raw(dir + "/q.f32", Q);
        read_raw(dir + "/k.f32", K);
        read_raw(dir + "/v.f32", V);
        read_raw(dir + "/m.f32", m);
        read_raw(dir + "/l.f32", l);
        FlashAttentionGradients r = flash_attention_backward(G, O, m, l, Q, K, V, scale);
        write_raw(dir + "/dq.f32", r.d_Q);
        write_raw(dir + "/dk.f32", r.d_K);
        write_raw(dir + "/dv.f32", r.d_V);
        std::cout << "OK\n";
        return 0;
    }
    return 2;
}
