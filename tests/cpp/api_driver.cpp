// api_driver.cpp -- exercises the C++ Tensor / autograd drop-in (libinferno.so).
//
// Device-parameterised in the way the reference's own tests are meant to be
// (InfernoTests/main.cpp:20-28 take an Inferno::Device): every case runs on
// Device::cpu() or Device::hip(0).
//
//   api_driver selftest <cpu|hip>
//       unit checks of views, element-wise ops, autograd, Softmax and attention;
//       prints PASS/FAIL lines, exit status = number of failures.
//   api_driver attn <dir> <B> <H> <T> <D> <f32|bf16> <cpu|hip> <causal> [qkv]
//       reads q.bin k.bin v.bin do.bin (fp32, [B,H,T,D]) from <dir>, runs
//       O = scaled_dot_product_attention(q, k, v) and (O * dO).backward(), writes
//       o.bin lse.bin dq.bin dk.bin dv.bin (fp32).  With "qkv", q, k and v are
//       views sliced out of one [B, T, 3C] projection tensor (the layout of
//       InfernoApp/main.cpp:712-734) and the gradients are read back from it.
//   api_driver softmax <dir> <rows> <cols> <f32|bf16> <cpu|hip> <axis>
//       reads x.bin g.bin ([rows, cols]); Y = Softmax(X, axis); (Y * G).backward();
//       writes y.bin dx.bin.
//   api_driver decode <dir> <B> <H> <Tk> <D> <f32|bf16> <cpu|hip>
//       reads q.bin kc.bin vc.bin, writes o.bin.
//   api_driver ckpt-save|ckpt-load <file> <cpu|hip>
//       Checkpoint round trips of a small module tree (see cmd_ckpt).
//   api_driver mask <dir> <cpu|hip>
//       triu / masked_fill cases on index-pattern inputs (see cmd_mask); writes
//       each result's raw bytes to <dir>/<case>.bin.
//   api_driver chain <dir> <B> <H> <T> <D> <cpu|hip>
//       the reference's unfused attention chain (InfernoApp/main.cpp:732-754)
//       on q.bin k.bin v.bin: kt = k^T contiguous, S = matmul(q, kt) * scale,
//       masked_fill(S, triu(ones[1,1,T,T] Int32, 1), -1e9f), Softmax, matmul with
//       v; writes y.bin and the mask's raw bytes mask.bin.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <functional>
#include <iostream>
#include <string>
#include <vector>

#include "inferno/inferno.h"

using namespace Inferno;

static std::vector<float> read_f32(const std::string& path, size_t n) {
    std::vector<float> v(n);
    std::ifstream f(path, std::ios::binary);
    if (!f.read(reinterpret_cast<char*>(v.data()), (std::streamsize)(n * 4))) throw Error("cannot read " + path);
    return v;
}

static void write_f32(const std::string& path, const std::vector<float>& v) {
    std::ofstream f(path, std::ios::binary);
    f.write(reinterpret_cast<const char*>(v.data()), (std::streamsize)(v.size() * 4));
}

static Device parse_dev(const std::string& s) { return s == "hip" ? Device::hip(0) : Device::cpu(); }
static DType parse_dt(const std::string& s) { return s == "bf16" ? DType::BFloat16 : DType::Float32; }

// ------------------------------------------------------------------ selftest
static int g_fail = 0;

static void check(bool ok, const std::string& name, const std::string& msg = "") {
    if (ok) {
        std::cout << "PASS " << name << "\n";
    } else {
        ++g_fail;
        std::cout << "FAIL " << name << (msg.empty() ? "" : ": " + msg) << "\n";
    }
}

static bool close(const std::vector<double>& a, const std::vector<double>& b, double tol) {
    if (a.size() != b.size()) return false;
    for (size_t i = 0; i < a.size(); ++i)
        if (std::fabs(a[i] - b[i]) > tol * (1.0 + std::fabs(b[i]))) return false;
    return true;
}

template <typename F>
static void run_case(const std::string& name, F f) {
    try {
        f();
    } catch (const std::exception& e) {
        check(false, name, std::string("exception: ") + e.what());
    }
}

static int selftest(Device dev) {
    run_case("create_and_transfer", [&] {
        Tensor t(DType::Float32, std::vector<float>{1, 2, 3, 4, 5, 6}, {2, 3}, "t", dev);
        check(t.shape() == std::vector<size_t>{2, 3} && t.numel() == 6 && t.is_contiguous(), "create_shape");
        check(close(t.to_host_double(), {1, 2, 3, 4, 5, 6}, 0), "create_values");
        check(t.device() == dev, "create_device");
        Tensor z = Tensor::zeros({3, 2}, DType::Float32, dev);
        check(close(z.to_host_double(), std::vector<double>(6, 0.0), 0), "zeros");
        Tensor o = Tensor::ones_like(t);
        check(close(o.to_host_double(), std::vector<double>(6, 1.0), 0), "ones_like");
        Tensor b(DType::BFloat16, std::vector<float>{1.0f, 1.00390625f, -2.5f}, {3}, "b", dev);
        check(close(b.to_host_double(), {1.0, 1.0, -2.5}, 0), "bf16_round_to_nearest_even");
    });
    run_case("views", [&] {
        Tensor t(DType::Float32, std::vector<float>{0, 1, 2, 3, 4, 5}, {2, 3}, "t", dev);
        Tensor tt = t.transpose(0, 1);
        check(tt.shape() == std::vector<size_t>{3, 2} && tt.strides() == std::vector<size_t>{1, 3} &&
                  !tt.is_contiguous(),
              "transpose_view");
        check(close(tt.contiguous().to_host_double(), {0, 3, 1, 4, 2, 5}, 0), "transpose_contiguous");
        bool threw = false;
        try {
            tt.reshape({6});
        } catch (const Error&) {
            threw = true;
        }
        check(threw, "reshape_noncontiguous_throws");
        check(close(t.reshape({3, 2}).to_host_double(), {0, 1, 2, 3, 4, 5}, 0), "reshape");
        Tensor s = t.slice(1, 1, 2);  // inclusive end
        check(s.shape() == std::vector<size_t>{2, 2} && close(s.to_host_double(), {1, 2, 4, 5}, 0), "slice_inclusive");
        check(close(t.transpose(-1, -2).to_host_double(), {0, 3, 1, 4, 2, 5}, 0), "transpose_negative_dims");
    });
    run_case("elementwise", [&] {
        Tensor a(DType::Float32, std::vector<float>{1, 2, 3}, {3}, "a", dev);
        Tensor b(DType::Float32, std::vector<float>{4, 5, 6}, {3}, "b", dev);
        check(close((a * b).to_host_double(), {4, 10, 18}, 0), "multiply");
        check(close((a + b).to_host_double(), {5, 7, 9}, 0), "add");
        check(close((a * 0.5f).to_host_double(), {0.5, 1, 1.5}, 0), "scalar_multiply");
        bool threw = false;
        try {
            Tensor c(DType::Float32, std::vector<float>{1, 2}, {2}, "c", dev);
            (void)(a * c);
        } catch (const Error&) {
            threw = true;
        }
        check(threw, "shape_mismatch_throws");
    });
    run_case("autograd_basic", [&] {
        Tensor x(DType::Float32, std::vector<float>{1, 2, 3}, {3}, "x", dev, true);
        Tensor y(DType::Float32, std::vector<float>{4, 5, 6}, {3}, "y", dev, true);
        Tensor r = x * y + x;  // dr/dx = y + 1, dr/dy = x
        r.backward();
        check(close(x.Getgrad().to_host_double(), {5, 6, 7}, 0), "grad_mul_add_x");
        check(close(y.Getgrad().to_host_double(), {1, 2, 3}, 0), "grad_mul_add_y");
        Tensor w(DType::Float32, std::vector<float>{2, 3}, {2}, "w", dev, true);
        Tensor seed(DType::Float32, std::vector<float>{10, 100}, {2}, "seed", dev);
        (w * w).backward(seed);  // explicit upstream gradient
        check(close(w.Getgrad().to_host_double(), {40, 600}, 0), "explicit_seed");
        {
            NoGradGuard ng;
            Tensor n = x * y;
            check(!n.requires_grad() && !GetImpl(n)->gradfn(), "no_grad_guard");
        }
    });
    run_case("autograd_views", [&] {
        Tensor x(DType::Float32, std::vector<float>{0, 1, 2, 3, 4, 5}, {2, 3}, "x", dev, true);
        Tensor g(DType::Float32, std::vector<float>{1, 2, 3, 4, 5, 6}, {3, 2}, "g", dev);
        Tensor t = x.transpose(0, 1).contiguous();
        (t * g).backward();
        check(close(x.Getgrad().to_host_double(), {1, 3, 5, 2, 4, 6}, 0), "transpose_contiguous_grad");
        Tensor x2(DType::Float32, std::vector<float>{0, 1, 2, 3, 4, 5}, {2, 3}, "x2", dev, true);
        Tensor s = x2.slice(1, 1, 2);
        Tensor gs(DType::Float32, std::vector<float>{7, 8, 9, 10}, {2, 2}, "gs", dev);
        (s.contiguous() * gs).backward();
        check(close(x2.Getgrad().to_host_double(), {0, 7, 8, 0, 9, 10}, 0), "slice_grad");
    });
    run_case("softmax", [&] {
        std::vector<float> xv = {1.f, 2.f, 3.f, -1e9f, 0.5f, 0.5f, 0.5f, 0.5f};
        Tensor x(DType::Float32, xv, {2, 4}, "x", dev, true);
        Tensor y = Softmax(x, -1);
        auto yh = y.to_host_double();
        double e1 = std::exp(-2.0), e2 = std::exp(-1.0), den = e1 + e2 + 1.0;
        check(close(yh, {e1 / den, e2 / den, 1.0 / den, 0.0, 0.25, 0.25, 0.25, 0.25}, 1e-6), "softmax_values");
        check(yh[3] == 0.0, "softmax_masked_exact_zero");
        check(y.requires_grad(), "softmax_output_requires_grad");
        Tensor g(DType::Float32, std::vector<float>{1, 0, -1, 2, 1, 2, 3, 4}, {2, 4}, "g", dev);
        (y * g).backward();
        std::vector<double> dx(8);
        for (int r = 0; r < 2; ++r) {
            double dot = 0;
            for (int c = 0; c < 4; ++c) dot += yh[r * 4 + c] * (double)(r == 0 ? std::vector<float>{1, 0, -1, 2}[c]
                                                                               : std::vector<float>{1, 2, 3, 4}[c]);
            for (int c = 0; c < 4; ++c) {
                const double gc = r == 0 ? std::vector<double>{1, 0, -1, 2}[c] : std::vector<double>{1, 2, 3, 4}[c];
                dx[r * 4 + c] = yh[r * 4 + c] * (gc - dot);
            }
        }
        check(close(x.Getgrad().to_host_double(), dx, 1e-6), "softmax_backward");
        Tensor xa(DType::Float32, std::vector<float>{1, 2, 3, 4, 5, 6}, {3, 2}, "xa", dev);
        Tensor ya = Softmax(xa, 0);  // non-last axis
        auto yah = ya.to_host_double();
        check(std::fabs(yah[0] + yah[2] + yah[4] - 1.0) < 1e-6 && std::fabs(yah[1] + yah[3] + yah[5] - 1.0) < 1e-6,
              "softmax_axis0");
    });
    run_case("attention_small", [&] {
        // T = 1: O = V exactly, dQ = dK = 0.
        Tensor q(DType::Float32, std::vector<float>(32, 0.3f), {1, 1, 1, 32}, "q", dev, true);
        Tensor k(DType::Float32, std::vector<float>(32, -0.7f), {1, 1, 1, 32}, "k", dev, true);
        std::vector<float> vv(32);
        for (int i = 0; i < 32; ++i) vv[i] = 0.1f * (float)i - 1.f;
        Tensor v(DType::Float32, vv, {1, 1, 1, 32}, "v", dev, true);
        Tensor o = scaled_dot_product_attention(q, k, v, true);
        check(close(o.to_host_double(), std::vector<double>(vv.begin(), vv.end()), 1e-6), "attention_T1_O_equals_V");
        check(o.requires_grad() && GetImpl(o)->gradfn() != nullptr, "attention_attaches_backward");
        o.backward();
        check(close(v.Getgrad().to_host_double(), std::vector<double>(32, 1.0), 1e-6), "attention_T1_dV_ones");
        auto dq = q.Getgrad().to_host_double();
        double mx = 0;
        for (double d : dq) mx = std::max(mx, std::fabs(d));
        check(mx < 1e-5, "attention_T1_dQ_zero");
        bool threw = false;
        try {
            Tensor k2(DType::Float32, std::vector<float>(48, 0.f), {1, 1, 1, 48}, "k2", dev);
            (void)scaled_dot_product_attention(q, k2, k2, true);
        } catch (const Error&) {
            threw = true;
        }
        check(threw, "attention_shape_mismatch_throws");
    });
    run_case("device_mismatch", [&] {
        if (!dev.is_hip()) return;
        Tensor a(DType::Float32, std::vector<float>{1, 2}, {2}, "a", dev);
        Tensor b(DType::Float32, std::vector<float>{1, 2}, {2}, "b", Device::cpu());
        bool threw = false;
        try {
            (void)(a * b);
        } catch (const Error&) {
            threw = true;
        }
        check(threw, "device_mismatch_throws");
    });
    run_case("argmax", [&] {
        // rows: plain, all equal (first index), a tie at 1 and 3, the maximum last
        Tensor x(DType::Float32, std::vector<float>{0, 5, 2, 1, 7, 7, 7, 7, 1, 9, 0, 9, -4, -3, -2, -1},
                 {2, 2, 4}, "x", dev);
        auto got = argmax(x).to_host_double();
        check(got == std::vector<double>{1, 0, 1, 3}, "argmax_rows_first_on_ties");
        // a [2, 1, 4] slice with strided rows (the last position of each sequence)
        auto last = argmax(x.slice(1, 1, 1)).to_host_double();
        check(last == std::vector<double>{0, 3}, "argmax_strided_rows");
        check(argmax(x).dtype() == DType::Int32 && argmax(x).shape() == std::vector<size_t>{2, 2},
              "argmax_shape_dtype");
    });
    std::cout << (g_fail ? "SELFTEST FAILED " : "SELFTEST OK ") << g_fail << "\n";
    return g_fail;
}

// --------------------------------------------------------------- attention
static int cmd_attn(int argc, char** argv) {
    if (argc < 10) throw Error("usage: attn <dir> B H T D f32|bf16 cpu|hip causal [qkv|qkvop]");
    const std::string dir = argv[2];
    const size_t B = std::stoul(argv[3]), H = std::stoul(argv[4]), T = std::stoul(argv[5]), D = std::stoul(argv[6]);
    const DType dt = parse_dt(argv[7]);
    const Device dev = parse_dev(argv[8]);
    const bool causal = std::stoi(argv[9]) != 0;
    // qkv: q, k, v as views of one [B, T, 3C] tensor into scaled_dot_product_attention;
    // qkvop: the same tensor through qkv_attention (the MultiHeadAttention op), y [B, T, C]
    const bool qkv_op = argc > 10 && std::string(argv[10]) == "qkvop";
    const bool qkv_layout = argc > 10 && (std::string(argv[10]) == "qkv" || qkv_op);
    const size_t n = B * H * T * D;
    auto qh = read_f32(dir + "/q.bin", n), kh = read_f32(dir + "/k.bin", n), vh = read_f32(dir + "/v.bin", n),
         gh = read_f32(dir + "/do.bin", n);
    Tensor dO(dt, gh, {B, H, T, D}, "dO", dev);
    Tensor q, k, v, qkv;
    if (!qkv_layout) {
        q = Tensor(dt, qh, {B, H, T, D}, "q", dev, true);
        k = Tensor(dt, kh, {B, H, T, D}, "k", dev, true);
        v = Tensor(dt, vh, {B, H, T, D}, "v", dev, true);
    } else {
        // [B, T, 3C] with C = H*D: q at columns [0, C), k at [C, 2C), v at [2C, 3C)
        const size_t C = H * D;
        std::vector<float> buf(B * T * 3 * C);
        for (size_t b = 0; b < B; ++b)
            for (size_t h = 0; h < H; ++h)
                for (size_t t = 0; t < T; ++t)
                    for (size_t d = 0; d < D; ++d) {
                        const size_t src = ((b * H + h) * T + t) * D + d;
                        const size_t dst = (b * T + t) * 3 * C + h * D + d;
                        buf[dst] = qh[src];
                        buf[dst + C] = kh[src];
                        buf[dst + 2 * C] = vh[src];
                    }
        qkv = Tensor(dt, buf, {B, T, 3 * C}, "qkv", dev, true);
        // slice (inclusive end, as InfernoApp/main.cpp:716-718) -> [B,T,H,D] -> [B,H,T,D], all views
        auto heads = [&](size_t c0) { return qkv.slice(2, c0, c0 + C - 1).unflatten(2, {H, D}).transpose(1, 2); };
        q = heads(0);
        k = heads(C);
        v = heads(2 * C);
    }
    Tensor lse, o;
    if (qkv_op) {
        Tensor y = qkv_attention(qkv, H, causal);  // [B, T, C]
        Tensor dOy;
        {
            NoGradGuard ng;
            dOy = dO.transpose(1, 2).contiguous().reshape({B, T, H * D});
        }
        (y * dOy).backward();
        NoGradGuard ng;
        o = y.unflatten(2, {H, D}).transpose(1, 2).contiguous();
        lse = Tensor::zeros({B, H, T}, DType::Float32, dev);
    } else {
        o = scaled_dot_product_attention_lse(q, k, v, causal, NAN, &lse);
        (o * dO).backward();
    }
    write_f32(dir + "/o.bin", o.to_host_float());
    write_f32(dir + "/lse.bin", lse.to_host_float());
    if (!qkv_layout) {
        write_f32(dir + "/dq.bin", q.Getgrad().to_host_float());
        write_f32(dir + "/dk.bin", k.Getgrad().to_host_float());
        write_f32(dir + "/dv.bin", v.Getgrad().to_host_float());
    } else {
        auto g = qkv.Getgrad().to_host_float();
        const size_t C = H * D;
        std::vector<float> dq(n), dk(n), dv(n);
        for (size_t b = 0; b < B; ++b)
            for (size_t h = 0; h < H; ++h)
                for (size_t t = 0; t < T; ++t)
                    for (size_t d = 0; d < D; ++d) {
                        const size_t dst = ((b * H + h) * T + t) * D + d;
                        const size_t src = (b * T + t) * 3 * C + h * D + d;
                        dq[dst] = g[src];
                        dk[dst] = g[src + C];
                        dv[dst] = g[src + 2 * C];
                    }
        write_f32(dir + "/dq.bin", dq);
        write_f32(dir + "/dk.bin", dk);
        write_f32(dir + "/dv.bin", dv);
    }
    std::cout << "attn ok\n";
    return 0;
}

static int cmd_softmax(int argc, char** argv) {
    if (argc < 8) throw Error("usage: softmax <dir> rows cols f32|bf16 cpu|hip axis");
    const std::string dir = argv[2];
    const size_t R = std::stoul(argv[3]), C = std::stoul(argv[4]);
    const DType dt = parse_dt(argv[5]);
    const Device dev = parse_dev(argv[6]);
    const int axis = std::stoi(argv[7]);
    Tensor x(dt, read_f32(dir + "/x.bin", R * C), {R, C}, "x", dev, true);
    Tensor g(dt, read_f32(dir + "/g.bin", R * C), {R, C}, "g", dev);
    Tensor y = Softmax(x, axis);
    (y * g).backward();
    write_f32(dir + "/y.bin", y.to_host_float());
    write_f32(dir + "/dx.bin", x.Getgrad().to_host_float());
    std::cout << "softmax ok\n";
    return 0;
}

// Softmax of a Float64 or Int32 tensor (the reference's other dispatchAny
// dtypes): x.bin holds doubles or int32s, g.bin the gradient in the output's
// dtype (Float64).  The backward runs where it can be seeded with g through
// (y * g).backward(): on the CPU device.
static int cmd_softmax_typed(int argc, char** argv) {
    if (argc < 8) throw Error("usage: softmax-typed <dir> rows cols f64|i32 cpu|hip axis");
    const std::string dir = argv[2];
    const size_t R = std::stoul(argv[3]), C = std::stoul(argv[4]);
    const std::string ts = argv[5];
    const Device dev = parse_dev(argv[6]);
    const int axis = std::stoi(argv[7]);
    auto raw = [&](const std::string& name, size_t bytes) {
        std::vector<char> v(bytes);
        std::ifstream f(dir + "/" + name, std::ios::binary);
        if (!f.read(v.data(), (std::streamsize)bytes)) throw Error("cannot read " + dir + "/" + name);
        return v;
    };
    auto save = [&](const std::string& name, const Tensor& t) {
        Tensor h = t.to(Device::cpu()).contiguous();
        std::ofstream f(dir + "/" + name, std::ios::binary);
        f.write(static_cast<const char*>(h.data_ptr()), (std::streamsize)(h.numel() * dtype_size(h.dtype())));
    };
    if (ts == "f64") {
        auto xb = raw("x.bin", R * C * 8);
        std::vector<double> xv(R * C);
        std::memcpy(xv.data(), xb.data(), xb.size());
        const bool grad = dev.is_cpu();
        Tensor x(DType::Float64, xv, {R, C}, "x", dev, grad);
        Tensor y = Softmax(x, axis);
        if (y.dtype() != DType::Float64) throw Error("softmax-typed: Float64 in, Float64 out expected");
        save("y.bin", y);
        if (grad) {
            auto gb = raw("g.bin", R * C * 8);
            std::vector<double> gv(R * C);
            std::memcpy(gv.data(), gb.data(), gb.size());
            Tensor g(DType::Float64, gv, {R, C}, "g", dev);
            (y * g).backward();
            if (x.Getgrad().dtype() != DType::Float64) throw Error("softmax-typed: Float64 gradient expected");
            save("dx.bin", x.Getgrad());
        }
    } else if (ts == "i32") {
        auto xb = raw("x.bin", R * C * 4);
        std::vector<int32_t> xv(R * C);
        std::memcpy(xv.data(), xb.data(), xb.size());
        Tensor x(DType::Int32, xv, {R, C}, "x", dev);
        Tensor y = Softmax(x, axis);
        if (y.dtype() != DType::Float32) throw Error("softmax-typed: Int32 in, Float32 out expected");
        save("y.bin", y);
    } else {
        throw Error("softmax-typed: f64 or i32");
    }
    std::cout << "softmax-typed ok\n";
    return 0;
}

static int cmd_decode(int argc, char** argv) {
    if (argc < 9) throw Error("usage: decode <dir> B H Tk D f32|bf16 cpu|hip");
    const std::string dir = argv[2];
    const size_t B = std::stoul(argv[3]), H = std::stoul(argv[4]), Tk = std::stoul(argv[5]), D = std::stoul(argv[6]);
    const DType dt = parse_dt(argv[7]);
    const Device dev = parse_dev(argv[8]);
    Tensor q(dt, read_f32(dir + "/q.bin", B * H * D), {B, H, 1, D}, "q", dev);
    Tensor kc(dt, read_f32(dir + "/kc.bin", B * H * Tk * D), {B, H, Tk, D}, "kc", dev);
    Tensor vc(dt, read_f32(dir + "/vc.bin", B * H * Tk * D), {B, H, Tk, D}, "vc", dev);
    write_f32(dir + "/o.bin", attention_decode(q, kc, vc).to_host_float());
    std::cout << "decode ok\n";
    return 0;
}

// ---------------------------------------------------------------- checkpoint
// A small module tree: Linear(4, 3) "fc", LayerNorm(3) "norm", Embedding(5, 4)
// "emb" in Float32 and a BFloat16 Linear(2, 2) "half", values fixed by seed.
struct CkptNet : Module {
    Linear fc;
    LayerNorm norm;
    Embedding emb;
    Linear half;
    explicit CkptNet(const Device& d)
        : fc(4, 3, d), norm(3, 1e-5f, d), emb(5, 4, d), half(2, 2, d, DType::BFloat16) {
        register_module("fc", &fc);
        register_module("norm", &norm);
        register_module("emb", &emb);
        register_module("half", &half);
    }
};

static void print_state(const StateDict& sd) {
    for (const auto& [name, t] : sd) {
        std::cout << name << " " << dtype_name(t.dtype());
        for (double v : t.to_host_double()) std::cout << " " << v;
        std::cout << "\n";
    }
}

//   api_driver ckpt-save <file> <cpu|hip>: seeded CkptNet on the device -> file; prints the state
//   api_driver ckpt-load <file> <cpu|hip>: file -> Checkpoint::load -> load_into a fresh CkptNet
//                                          on the device; prints the module's state
static int cmd_ckpt(int argc, char** argv) {
    if (argc < 4) throw Error("usage: api_driver ckpt-save|ckpt-load <file> <cpu|hip>");
    const std::string mode = argv[1], path = argv[2];
    const Device dev = parse_dev(argv[3]);
    if (mode == "ckpt-save") {
        RandomGenerator::initializeWithSeed(123);
        CkptNet net(dev);
        Checkpoint c;
        c.set_state_dict(net.state_dict());
        c.save(path);
        print_state(net.state_dict());
    } else {
        RandomGenerator::initializeWithSeed(999);
        CkptNet net(dev);
        Checkpoint c;
        Checkpoint loaded = c.load(path);
        Checkpoint::load_into(net, loaded.state_dict());
        print_state(net.state_dict());
    }
    return 0;
}

static void write_raw(const std::string& path, const Tensor& t) {
    const Tensor h = t.to(Device::cpu());
    if (!h.is_contiguous()) throw Error("write_raw: expected a dense tensor");
    std::ofstream f(path, std::ios::binary);
    f.write(static_cast<const char*>(h.data_ptr()), (std::streamsize)(h.numel() * dtype_size(h.dtype())));
}

// Index-pattern input: element i = i * step + base, converted to dt.
static Tensor pattern(DType dt, const std::vector<size_t>& shape, float step, float base, Device dev) {
    size_t n = 1;
    for (size_t d : shape) n *= d;
    std::vector<float> v(n);
    for (size_t i = 0; i < n; ++i) v[i] = (float)i * step + base;
    return Tensor(dt, v, shape, "pattern", dev);
}

static int cmd_mask(int argc, char** argv) {
    if (argc < 4) throw Error("usage: mask <dir> <cpu|hip>");
    const std::string dir = argv[2];
    const Device dev = parse_dev(argv[3]);
    const Tensor a = pattern(DType::Float32, {2, 3, 5, 7}, 0.5f, -10.f, dev);
    const Tensor at = a.transpose(2, 3);  // [2, 3, 7, 5], a strided view
    for (int dg : {-2, 0, 1, 3}) {
        write_raw(dir + "/triu_f32_" + std::to_string(dg + 2) + ".bin", triu(a, dg));
        write_raw(dir + "/triu_f32t_" + std::to_string(dg + 2) + ".bin", triu(at, dg));
    }
    const Tensor ones(DType::Int32, std::vector<int>(6 * 9, 1), {1, 1, 6, 9}, "ones", dev);
    const Tensor causal = triu(ones, 1);
    write_raw(dir + "/triu_i32.bin", causal);
    write_raw(dir + "/triu_bf16.bin", triu(pattern(DType::BFloat16, {4, 6}, 0.25f, -3.f, dev), -1));
    const Tensor m57 = triu(Tensor(DType::Int32, std::vector<int>(5 * 7, 1), {5, 7}, "ones57", dev), 1);
    write_raw(dir + "/mf_f32.bin", masked_fill(a, m57, -1e9f));
    const Tensor m75 = triu(Tensor(DType::Int32, std::vector<int>(7 * 5, 1), {7, 5}, "ones75", dev), 0);
    write_raw(dir + "/mf_f32t.bin", masked_fill(at, m75, 2.5f));
    write_raw(dir + "/mf_i8.bin", masked_fill(a, pattern(DType::Int8, {1, 7}, 1.f, -3.f, dev), 7.f));
    write_raw(dir + "/mf_bool.bin", masked_fill(a, pattern(DType::Bool, {3, 1, 1}, 1.f, 0.f, dev), -1.f));
    std::vector<int> every3(2 * 5 * 7);
    for (size_t i = 0; i < every3.size(); ++i) every3[i] = i % 3 == 0 ? 1 : 0;
    write_raw(dir + "/mf_bf16.bin", masked_fill(pattern(DType::BFloat16, {2, 3, 5, 7}, 0.25f, -7.f, dev),
                                                Tensor(DType::Int32, every3, {2, 1, 5, 7}, "every3", dev), -1e9f));
    write_raw(dir + "/mf_i32.bin",
              masked_fill(pattern(DType::Int32, {4, 6}, 3.f, -20.f, dev), pattern(DType::Bool, {6}, 1.f, -2.f, dev),
                          -3.7f));
    return 0;
}

static int cmd_chain(int argc, char** argv) {
    if (argc < 8) throw Error("usage: chain <dir> B H T D cpu|hip");
    const std::string dir = argv[2];
    const size_t B = std::stoul(argv[3]), H = std::stoul(argv[4]), T = std::stoul(argv[5]), D = std::stoul(argv[6]);
    const Device dev = parse_dev(argv[7]);
    const size_t n = B * H * T * D;
    NoGradGuard ng;
    const Tensor q(DType::Float32, read_f32(dir + "/q.bin", n), {B, H, T, D}, "q", dev);
    const Tensor k(DType::Float32, read_f32(dir + "/k.bin", n), {B, H, T, D}, "k", dev);
    const Tensor v(DType::Float32, read_f32(dir + "/v.bin", n), {B, H, T, D}, "v", dev);
    const Tensor kt = k.transpose(-1, -2).contiguous();
    Tensor scores = matmul(q, kt, "QK ^ T");
    const float scale = 1.0f / std::sqrt(static_cast<float>(D));
    scores = scores * scale;
    const Tensor ones(DType::Int32, std::vector<int>(T * T, 1), {1, 1, T, T}, "causal_mask_ones", dev);
    const Tensor mask = triu(ones, 1);
    scores = masked_fill(scores, mask, -1e9f);
    const Tensor attn = Softmax(scores, -1).contiguous();
    const Tensor y = matmul(attn, v, "attn@V");
    write_raw(dir + "/y.bin", y);
    write_raw(dir + "/mask.bin", mask);
    return 0;
}

int main(int argc, char** argv) {
    if (argc < 2) {
        std::cerr << "usage: api_driver selftest|attn|softmax|decode ...\n";
        return 2;
    }
    try {
        const std::string cmd = argv[1];
        if (cmd == "selftest") return selftest(parse_dev(argc > 2 ? argv[2] : "cpu"));
        if (cmd == "attn") return cmd_attn(argc, argv);
        if (cmd == "softmax") return cmd_softmax(argc, argv);
        if (cmd == "softmax-typed") return cmd_softmax_typed(argc, argv);
        if (cmd == "decode") return cmd_decode(argc, argv);
        if (cmd == "ckpt-save" || cmd == "ckpt-load") return cmd_ckpt(argc, argv);
        if (cmd == "mask") return cmd_mask(argc, argv);
        if (cmd == "chain") return cmd_chain(argc, argv);
        std::cerr << "unknown command " << cmd << "\n";
        return 2;
    } catch (const std::exception& e) {
        std::cerr << "error: " << e.what() << "\n";
        return 3;
    }
}
