// soklyn_tool — command-line driver of the C++ host API (soklyn.hpp).
//
//   soklyn_tool selftest                      host-only checks (no GPU needed)
//   soklyn_tool chacha ROUNDS KEYHEX COUNTER NBLOCKS
//                                             ChaCha keystream words (hex), 64-bit counter
//   soklyn_tool pcg32 SEED SEQ N              pcg-c's pcg32 sequence (hex)
//   soklyn_tool init KIND SEED FACTOR FAN_IN FAN_OUT LEN
//                                             initialiser output as f32 bit patterns (hex);
//                                             KIND = he_normal | he_uniform | xavier_normal |
//                                             xavier_uniform
//   soklyn_tool ids                           tensor ids taken by fp32 / fp16 training and
//                                             inference blocks (needs a GPU)
//   soklyn_tool train DIR                     FeedForwardNetwork training steps described by
//                                             DIR/spec.txt on DIR/x.bin, DIR/t.bin (needs a GPU);
//                                             then saves DIR/net.safetensors, loads it back and
//                                             checks the reloaded network
//   soklyn_tool convert DIR K N BATCH SEED    DenseBlock<f32>::convert_f16, one fp16 Adam step
//                                             (MSE on DIR/x.bin, DIR/t.bin), convert_f32, one fp32
//                                             forward; dumps every stage into DIR (needs a GPU)
//   soklyn_tool sched cosine MIN MAX TOTAL WARMUP N | sched exp LR FACTOR N |
//              sched plateau PATIENCE min|max FACTOR MIN_LR RESET_LR V...
//                                             learning-rate schedules (no GPU): the rate after
//                                             construction (plateau: after reset) and after each
//                                             step, as f32 bit patterns (hex)
//   soklyn_tool st-demo FILE                  write a synthetic safetensors file (no GPU)
//   soklyn_tool st-dump FILE                  print a safetensors file: metadata, then per tensor
//                                             name, dtype, shape and the bytes in hex (no GPU)
//
// `train` writes, per layer i: w<i>_init.bin (initial weights as f32), and after
// the last step out<i>, w<i>, master_w<i> (fp16), b<i>, dv_w<i>, dm_w<i>, dv_b<i>,
// grad<i>, d_prenorm<i>, mask<i> as raw little-endian f32; ids.txt holds each
// layer's weight tensor id (the dropout seed is scramble_seed(step, id)).
#include <cfloat>
#include <cinttypes>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <algorithm>
#include <map>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

#include "safetensors.hpp"
#include "scheduler.hpp"
#include "soklyn.hpp"

using namespace soklyn;

namespace {

int usage() {
    std::fprintf(stderr, "usage: soklyn_tool selftest | chacha R KEYHEX CTR N | init KIND SEED FACTOR FIN FOUT LEN | "
                         "ids | train DIR | convert DIR K N BATCH SEED | sched ... | st-demo FILE | st-dump FILE\n");
    return 2;
}

int selftest() {
    int bad = 0;
    // every binary16 value survives f16 -> f32 -> f16 (NaNs stay NaN)
    for (uint32_t b = 0; b < 65536; ++b) {
        f16 h;
        h.bits = static_cast<uint16_t>(b);
        const float f = h.to_f32();
        const f16 back = f16::from_f32(f);
        const bool nan = ((b >> 10) & 0x1f) == 0x1f && (b & 0x3ff);
        if (nan ? !(((back.bits >> 10) & 0x1f) == 0x1f && (back.bits & 0x3ff)) : back.bits != b) {
            if (bad++ < 5) std::fprintf(stderr, "f16 round trip %04x -> %04x\n", b, back.bits);
        }
    }
    // ties to even at the subnormal and normal boundaries, overflow
    struct Case { float v; uint16_t bits; } cases[] = {
        {1.0f, 0x3c00}, {65504.0f, 0x7bff}, {65519.99f, 0x7bff}, {65520.0f, 0x7c00}, {-65520.0f, 0xfc00},
        {5.9604644775390625e-08f, 0x0001}, {2.98023223876953125e-08f, 0x0000}, {2.9802326e-08f, 0x0001},
        {8.940696716308594e-08f, 0x0002}, {1.0009765625f, 0x3c01}, {1.00048828125f, 0x3c00},
        {1.00146484375f, 0x3c02}, {6.097555160522461e-05f, 0x03ff}, {6.103515625e-05f, 0x0400},
    };
    for (const Case &c : cases) {
        const f16 h = f16::from_f32(c.v);
        if (h.bits != c.bits) {
            std::fprintf(stderr, "f16::from_f32(%.10g) = %04x, want %04x\n", c.v, h.bits, c.bits);
            ++bad;
        }
    }
    // status codes map onto the reference's Error variants
    const std::pair<int32_t, ErrorKind> kinds[] = {
        {SKL_ERR_INVALID_CONFIGURATION, ErrorKind::InvalidConfiguration},
        {SKL_ERR_TRAINING_MODE_REQUIRED, ErrorKind::TrainingModeRequired},
        {SKL_ERR_ALLOCATION_LIMIT, ErrorKind::AllocationLimitExceeded},
        {SKL_ERR_MISMATCHED_DIMENSIONS, ErrorKind::MismatchedDimensions},
        {SKL_ERR_INVALID_BATCH_SIZE, ErrorKind::InvalidBatchSize},
        {SKL_ERR_NO_DEVICE, ErrorKind::NoDevice},
        {1, ErrorKind::DriverError},
    };
    for (const auto &k : kinds) {
        try {
            check(k.first, "selftest");
            ++bad;
        } catch (const Error &e) {
            if (e.kind() != k.second || e.status() != k.first) ++bad;
        }
    }
    try {
        check(SKL_OK, "selftest");
    } catch (...) {
        ++bad;
    }
    if (scramble_seed(1, 7) != skl_scramble_seed(1, 7)) ++bad;
    std::printf("%s\n", bad ? "FAIL" : "OK");
    return bad ? 1 : 0;
}

int chacha(int rounds, const char *keyhex, uint64_t counter, int nblocks) {
    uint32_t k[8] = {};
    if (std::strlen(keyhex) != 64) return usage();
    for (int i = 0; i < 32; ++i) {
        unsigned v = 0;
        std::sscanf(keyhex + 2 * i, "%2x", &v);
        k[i / 4] |= static_cast<uint32_t>(v) << (8 * (i % 4));
    }
    for (int b = 0; b < nblocks; ++b) {
        uint32_t out[16];
        ChaCha8Rng::block(k, counter + b, rounds, out);
        for (int i = 0; i < 16; ++i) std::printf("%08x%c", out[i], i == 15 ? '\n' : ' ');
    }
    return 0;
}

// pcg-c's pcg32_srandom_r / pcg32_random_r sequence (outputs from the state
// before each step), used to pin the XSH-RR output and the LCG multiplier.
int pcg32(uint64_t seed, uint64_t seq, int n) {
    const uint64_t inc = (seq << 1u) | 1u;
    uint64_t state = 0;
    state = state * PCG32_MULTIPLIER + inc;
    state += seed;
    state = state * PCG32_MULTIPLIER + inc;
    for (int i = 0; i < n; ++i) {
        const uint64_t old = state;
        state = old * PCG32_MULTIPLIER + inc;
        std::printf("%08x%c", pcg32_xsh_rr(old), i + 1 == n ? '\n' : ' ');
    }
    return 0;
}

int init_dump(const std::string &kind, uint64_t seed, float factor, size_t fan_in, size_t fan_out, size_t len) {
    std::unique_ptr<InitFunc> f;
    if (kind == "he_normal") f.reset(new InitHeNormalFunc(seed, factor));
    else if (kind == "he_uniform") f.reset(new InitHeUniformFunc(seed, factor));
    else if (kind == "xavier_normal") f.reset(new InitXavierNormalFunc(seed, factor));
    else if (kind == "xavier_uniform") f.reset(new InitXavierUniformFunc(seed, factor));
    else return usage();
    const std::vector<float> v = f->init_f32(fan_in, fan_out, len);
    for (size_t i = 0; i < v.size(); ++i) {
        uint32_t x;
        std::memcpy(&x, &v[i], 4);
        std::printf("%08x%c", x, (i % 8 == 7 || i + 1 == v.size()) ? '\n' : ' ');
    }
    return 0;
}

// ---- safetensors ------------------------------------------------------------------------------
int st_demo(const std::string &path) {
    SafetensorFile f;
    SafetensorWriter &w = const_cast<SafetensorWriter &>(f.writer());
    std::vector<float> a(6);
    for (int i = 0; i < 6; ++i) a[i] = 0.5f * static_cast<float>(i) - 1.25f;
    std::vector<uint8_t> ab(a.size() * 4);
    std::memcpy(ab.data(), a.data(), ab.size());
    w.pass("layer1.w", {2, 3}, ab, Precision::FP32);
    std::vector<uint16_t> h = {f16::from_f32(1.5f).bits, f16::from_f32(-2.0f).bits, f16::from_f32(0.1f).bits,
                               f16::from_f32(65504.0f).bits, f16::from_f32(-0.0f).bits};
    std::vector<uint8_t> hb(h.size() * 2);
    std::memcpy(hb.data(), h.data(), hb.size());
    w.pass("alpha", {5}, hb, Precision::FP16);
    const float sc = 3.25f;
    std::vector<uint8_t> sb(4);
    std::memcpy(sb.data(), &sc, 4);
    w.pass("scalar", {}, sb, Precision::FP32);
    w.pass("empty", {0, 3}, {}, Precision::FP32);
    f.pass_metadata("name", "demo \"quoted\" \\ / \xc3\xa9 \t tab\n line");
    f.pass_metadata("epoch", "7");
    f.pass_metadata("name", "demo \"quoted\" \\ / \xc3\xa9 \t tab\n line\x01");   // replaces in place
    f.save(path);
    return 0;
}

int st_dump(const std::string &path) {
    const SafetensorFile f = SafetensorFile::read(path);
    std::vector<std::pair<std::string, std::string>> md = f.get_metadata();
    std::sort(md.begin(), md.end());
    for (const auto &kv : md) {
        JsonValue k, v;
        k.kind = v.kind = JsonValue::Kind::String;
        k.text = kv.first;
        v.text = kv.second;
        std::printf("meta %s %s\n", k.to_compact().c_str(), v.to_compact().c_str());
    }
    std::vector<const SafetensorDescriptor *> ds;
    for (const SafetensorDescriptor &d : f.writer().get_descriptors()) ds.push_back(&d);
    std::sort(ds.begin(), ds.end(), [](auto *a, auto *b) { return a->name < b->name; });
    for (const SafetensorDescriptor *d : ds) {
        std::printf("tensor %s %s", d->name.c_str(), d->precision == Precision::FP32 ? "F32" : "F16");
        std::printf(" [");
        for (size_t i = 0; i < d->shape.size(); ++i) std::printf(i ? ",%zu" : "%zu", d->shape[i]);
        std::printf("] ");
        for (uint8_t b : d->data) std::printf("%02x", b);
        std::printf("\n");
    }
    return 0;
}

template <class T> size_t block_ids(const GpuContext &ctx, bool training) {
    InitZeroFunc zero;
    const size_t before = peek_tensor_id_counter();
    DenseBlock<T> b = DenseBlock<T>::new_with_config(ctx, training, 8, 4, 16, zero, LayerInitConfig{});
    const size_t after = peek_tensor_id_counter();
    if (b.get_weights().get_id() != before) return 0;   // the weight is the block's first tensor
    return after - before;
}

int ids() {
    GpuContext ctx;
    std::printf("f32_train %zu\nf16_train %zu\nf32_infer %zu\nf16_infer %zu\n", block_ids<float>(ctx, true),
                block_ids<f16>(ctx, true), block_ids<float>(ctx, false), block_ids<f16>(ctx, false));
    return 0;
}

// ---- train ----------------------------------------------------------------------------------
std::map<std::string, std::string> read_spec(const std::string &path) {
    std::ifstream in(path);
    if (!in) throw std::runtime_error("cannot read " + path);
    std::map<std::string, std::string> m;
    std::string line;
    while (std::getline(in, line)) {
        const size_t eq = line.find('=');
        if (line.empty() || line[0] == '#' || eq == std::string::npos) continue;
        m[line.substr(0, eq)] = line.substr(eq + 1);
    }
    return m;
}

std::vector<float> read_f32(const std::string &path, size_t n) {
    std::vector<float> v(n);
    std::ifstream in(path, std::ios::binary);
    if (!in.read(reinterpret_cast<char *>(v.data()), static_cast<std::streamsize>(n * 4)))
        throw std::runtime_error("short read: " + path);
    return v;
}

void write_f32(const std::string &path, const std::vector<float> &v) {
    std::ofstream out(path, std::ios::binary);
    out.write(reinterpret_cast<const char *>(v.data()), static_cast<std::streamsize>(v.size() * 4));
}

template <class T, size_t R> std::vector<float> host_f32(const GpuContext &ctx, const Tensor<T, R> &t) {
    const std::vector<T> v = t.download(ctx);
    std::vector<float> f(v.size());
    for (size_t i = 0; i < v.size(); ++i) f[i] = PrecisionType<T>::to_f32(v[i]);
    return f;
}

Optimiser parse_opt(const std::map<std::string, std::string> &s) {
    if (s.at("opt") == "adam")
        return Optimiser::adam(std::stof(s.at("m")), std::stof(s.at("v")), std::stof(s.at("eps")));
    return Optimiser::sgd(std::stof(s.at("v")), s.at("nesterov") == "1");
}

template <class T> int train(const std::string &dir, const std::map<std::string, std::string> &s) {
    std::vector<size_t> dims;
    {
        std::stringstream ss(s.at("dims"));
        std::string tok;
        while (std::getline(ss, tok, ',')) dims.push_back(std::stoul(tok));
    }
    const size_t batch = std::stoul(s.at("batch")), steps = std::stoul(s.at("steps"));
    const size_t L = dims.size() - 1;
    GpuContext ctx;

    LayerInitConfig hidden;
    hidden.normalisation = static_cast<Normalisation>(std::stoul(s.at("norm")));
    hidden.activation = {static_cast<Activation::Kind>(std::stoul(s.at("act"))), std::stof(s.at("leaky"))};
    hidden.mask_coeff = std::stof(s.at("mask_coeff"));
    LayerInitConfig head;   // output layer: Identity, no norm, no dropout
    InitHeNormalFunc init(std::stoull(s.at("init_seed")), 1.0f);
    std::vector<DenseBlock<T>> layers;
    for (size_t i = 0; i < L; ++i)
        layers.push_back(DenseBlock<T>::new_with_config(ctx, true, dims[i], dims[i + 1], batch, init,
                                                        i + 1 < L ? hidden : head));
    {
        std::ofstream ids(dir + "/ids.txt");
        for (size_t i = 0; i < L; ++i) {
            ids << layers[i].get_weights().get_id() << "\n";
            write_f32(dir + "/w" + std::to_string(i) + "_init.bin", host_f32(ctx, layers[i].get_weights()));
        }
    }
    FeedForwardNetwork<T> net(std::move(layers), dims[0]);

    auto to_t = [](const std::vector<float> &f) {
        std::vector<T> v(f.size());
        for (size_t i = 0; i < f.size(); ++i) v[i] = PrecisionType<T>::from_f32(f[i]);
        return v;
    };
    const Tensor2D<T> x = Tensor2D<T>::from_cpu_vector(ctx, to_t(read_f32(dir + "/x.bin", batch * dims[0])),
                                                       {batch, dims[0]});
    const Tensor2D<T> t = Tensor2D<T>::from_cpu_vector(ctx, to_t(read_f32(dir + "/t.bin", batch * dims[L])),
                                                       {batch, dims[L]});
    const LossConfig loss{static_cast<LossFunc>(std::stoul(s.at("loss"))),
                          {static_cast<Activation::Kind>(std::stoul(s.at("loss_act"))), 0.0f}};
    MultiLayerTrainContext tc{std::vector<Optimiser>(L, parse_opt(s)), std::vector<Optimiser>(L, parse_opt(s)), batch,
                              std::stof(s.at("lr")), FLT_MAX};
    const bool dropout = s.at("dropout") == "1";
    for (size_t step = 1; step <= steps; ++step) {
        const std::vector<const Tensor2D<T> *> outs = net.forward(ctx, x, batch, dropout, step);
        net.backward(ctx, outs, t, x, loss, tc, step);
    }
    ctx.synchronize();
    for (size_t i = 0; i < L; ++i) {
        const DenseBlock<T> &b = net.get_layers()[i];
        const std::string n = std::to_string(i);
        write_f32(dir + "/out" + n + ".bin", host_f32(ctx, b.get_outputs()));
        write_f32(dir + "/w" + n + ".bin", host_f32(ctx, b.get_weights()));
        if (b.get_master_weights()) write_f32(dir + "/master_w" + n + ".bin", host_f32(ctx, *b.get_master_weights()));
        write_f32(dir + "/b" + n + ".bin", host_f32(ctx, b.get_biases()));
        write_f32(dir + "/dv_w" + n + ".bin", host_f32(ctx, b.get_dv_weights()));
        write_f32(dir + "/dm_w" + n + ".bin", host_f32(ctx, b.get_dm_weights()));
        write_f32(dir + "/dv_b" + n + ".bin", host_f32(ctx, b.get_dv_biases()));
        write_f32(dir + "/grad" + n + ".bin", host_f32(ctx, b.get_grads()));
        write_f32(dir + "/d_prenorm" + n + ".bin", host_f32(ctx, b.get_delta_prenorm_out()));
        write_f32(dir + "/mask" + n + ".bin", host_f32(ctx, b.get_masks()));
    }
    // checkpoint round trip (save.rs): save, read back into blocks, compare every
    // tensor bit for bit, then the reloaded network's forward against the original's
    {
        SafetensorFile sf = SafetensorFile::from_ffn(ctx, net);
        sf.pass_metadata("steps", std::to_string(steps));
        sf.save(dir + "/net.safetensors");
        std::vector<DenseBlock<T>> back =
            SafetensorFile::read(dir + "/net.safetensors").template into_blocks<T>(ctx, true, batch);
        if (back.size() != L) throw std::runtime_error("round trip: layer count");
        auto same = [&](const auto &a, const auto &b, const char *what, size_t i) {
            const auto va = a.download(ctx), vb = b.download(ctx);
            if (va.size() != vb.size() || std::memcmp(va.data(), vb.data(), va.size() * sizeof(va[0])) != 0)
                throw std::runtime_error(std::string("round trip: ") + what + " of layer " + std::to_string(i));
        };
        for (size_t i = 0; i < L; ++i) {
            const DenseBlock<T> &o = net.get_layers()[i];
            DenseBlock<T> &r = back[i];
            same(o.get_weights(), r.get_weights(), "w", i);
            same(o.get_biases(), r.get_biases(), "b", i);
            same(o.get_norm_weights(), r.get_norm_weights(), "norm_w", i);
            same(o.get_norm_biases(), r.get_norm_biases(), "norm_b", i);
            same(o.get_dv_weights(), r.get_dv_weights(), "dv_w", i);
            same(o.get_dm_weights(), r.get_dm_weights(), "dm_w", i);
            same(o.get_dv_norm_weights(), r.get_dv_norm_weights(), "dv_norm_w", i);
            same(o.get_dm_norm_biases(), r.get_dm_norm_biases(), "dm_norm_b", i);
            if (o.get_master_weights()) same(*o.get_master_weights(), *r.get_master_weights(), "master_w", i);
            if (o.get_master_norm_weights())
                same(*o.get_master_norm_weights(), *r.get_master_norm_weights(), "master_norm_w", i);
            // loaded blocks carry the default layer config (save.rs:567-572): set it again
            r.set_normalisation(o.get_normalisation());
            r.set_activation(o.get_activation());
            r.set_mask_coeff(o.get_mask_coeff());
        }
        FeedForwardNetwork<T> net2(std::move(back), dims[0]);
        const std::vector<float> y1 = host_f32(ctx, *net.forward(ctx, x, batch, false, steps + 1).back());
        const std::vector<float> y2 = host_f32(ctx, *net2.forward(ctx, x, batch, false, steps + 1).back());
        if (std::memcmp(y1.data(), y2.data(), y1.size() * 4) != 0) throw std::runtime_error("round trip: forward");
        std::printf("checkpoint round trip OK\n");
    }
    std::printf("trained %zu steps\n", steps);
    return 0;
}

// ---- sched: learning-rate schedules (scheduler.rs) -------------------------------------------
void print_bits(float v, bool last) {
    uint32_t x;
    std::memcpy(&x, &v, 4);
    std::printf("%08x%c", x, last ? '\n' : ' ');
}

int sched(int argc, char **argv) {
    const std::string kind = argv[2];
    if (kind == "cosine" && argc == 8) {
        CosineDecayLR s(std::strtof(argv[3], nullptr), std::strtof(argv[4], nullptr), std::strtoul(argv[5], nullptr, 10),
                        std::strtoul(argv[6], nullptr, 10));
        const size_t n = std::strtoul(argv[7], nullptr, 10);
        print_bits(s.get_learning_rate(), n == 0);
        for (size_t i = 0; i < n; ++i) print_bits(s.step(), i + 1 == n);
        s.reset();
        std::printf("reset ");
        print_bits(s.get_learning_rate(), true);
        return 0;
    }
    if (kind == "exp" && argc == 6) {
        ExponentialLR s(std::strtof(argv[3], nullptr), std::strtof(argv[4], nullptr));
        const size_t n = std::strtoul(argv[5], nullptr, 10);
        print_bits(s.get_learning_rate(), n == 0);
        for (size_t i = 0; i < n; ++i) print_bits(s.step(), i + 1 == n);
        s.reset();
        std::printf("reset ");
        print_bits(s.get_learning_rate(), true);
        return 0;
    }
    if (kind == "plateau" && argc >= 8) {
        const std::string mode = argv[4];
        ReduceLROnPlateauScheduler s(std::strtoul(argv[3], nullptr, 10),
                                     mode == "max" ? SchedulerMode::Maximize : SchedulerMode::Minimize,
                                     std::strtof(argv[5], nullptr), std::strtof(argv[6], nullptr));
        print_bits(s.get_learning_rate(), false);
        s.reset(std::strtof(argv[7], nullptr));
        print_bits(s.get_learning_rate(), argc == 8);
        for (int i = 8; i < argc; ++i) print_bits(s.step(std::strtof(argv[i], nullptr)), i + 1 == argc);
        return 0;
    }
    return usage();
}

// ---- convert: DenseBlock<f32>::convert_f16 -> one training step -> convert_f32 ---------------
// (mlp.rs:835-888).  One RMSNorm + SiLU block K -> N, He-normal init from init_seed; x
// [batch x K] and the MSE target t [batch x N] are read from dir.  Dumps every stage so the
// caller can check the casts bit for bit and the step against the oracle.
int convert(const std::string &dir, size_t K, size_t N, size_t batch, uint64_t init_seed) {
    GpuContext ctx;
    InitHeNormalFunc init(init_seed, 1.0f);
    LayerInitConfig cfg;
    cfg.normalisation = Normalisation::RMSNorm;
    cfg.activation = Activation::silu();
    DenseBlock<float> b32 = DenseBlock<float>::new_with_config(ctx, true, K, N, batch, init, cfg);
    write_f32(dir + "/w32_init.bin", host_f32(ctx, b32.get_weights()));
    write_f32(dir + "/mask32_init.bin", host_f32(ctx, b32.get_masks()));

    DenseBlock<f16> b16 = std::move(b32).convert_f16(ctx);
    write_f32(dir + "/w16.bin", host_f32(ctx, b16.get_weights()));
    write_f32(dir + "/master_w16.bin", host_f32(ctx, b16.get_master_weights().value()));
    write_f32(dir + "/master_norm_w16.bin", host_f32(ctx, b16.get_master_norm_weights().value()));
    write_f32(dir + "/norm_w16.bin", host_f32(ctx, b16.get_norm_weights()));
    write_f32(dir + "/mask16.bin", host_f32(ctx, b16.get_masks()));

    auto to_h = [](const std::vector<float> &f) {
        std::vector<f16> v(f.size());
        for (size_t i = 0; i < f.size(); ++i) v[i] = PrecisionType<f16>::from_f32(f[i]);
        return v;
    };
    const Tensor2D<f16> x = Tensor2D<f16>::from_cpu_vector(ctx, to_h(read_f32(dir + "/x.bin", batch * K)), {batch, K});
    const Tensor2D<f16> t = Tensor2D<f16>::from_cpu_vector(ctx, to_h(read_f32(dir + "/t.bin", batch * N)), {batch, N});
    const Optimiser adam = Optimiser::adam(0.9f, 0.999f, 1e-8f);
    const TrainContext tc{&adam, &adam, batch, 1e-3f, FLT_MAX};
    b16.forward(ctx, x, batch, false, 1);
    b16.compute_loss(ctx, t, LossConfig{LossFunc::MeanSquareLoss, Activation::identity()});
    b16.backward_output(ctx, x, tc, 1);
    ctx.synchronize();
    write_f32(dir + "/out16.bin", host_f32(ctx, b16.get_outputs()));
    write_f32(dir + "/d_prenorm16.bin", host_f32(ctx, b16.get_delta_prenorm_out()));
    write_f32(dir + "/w16_step.bin", host_f32(ctx, b16.get_weights()));
    write_f32(dir + "/master_w16_step.bin", host_f32(ctx, b16.get_master_weights().value()));
    write_f32(dir + "/master_norm_w16_step.bin", host_f32(ctx, b16.get_master_norm_weights().value()));
    write_f32(dir + "/master_b16_step.bin", host_f32(ctx, b16.get_master_biases().value()));
    write_f32(dir + "/master_norm_b16_step.bin", host_f32(ctx, b16.get_master_norm_biases().value()));
    write_f32(dir + "/dm_w16_step.bin", host_f32(ctx, b16.get_dm_weights()));
    write_f32(dir + "/dv_w16_step.bin", host_f32(ctx, b16.get_dv_weights()));

    DenseBlock<float> back = std::move(b16).convert_f32(ctx);
    write_f32(dir + "/w32_back.bin", host_f32(ctx, back.get_weights()));
    write_f32(dir + "/b32_back.bin", host_f32(ctx, back.get_biases()));
    write_f32(dir + "/norm_w32_back.bin", host_f32(ctx, back.get_norm_weights()));
    write_f32(dir + "/norm_b32_back.bin", host_f32(ctx, back.get_norm_biases()));
    write_f32(dir + "/dm_w32_back.bin", host_f32(ctx, back.get_dm_weights()));
    write_f32(dir + "/dv_w32_back.bin", host_f32(ctx, back.get_dv_weights()));
    write_f32(dir + "/out32_back.bin", host_f32(ctx, back.get_outputs()));
    // the converted block keeps working in fp32: one forward on the fp16 inputs
    const std::vector<float> xf = read_f32(dir + "/x.bin", batch * K);
    std::vector<float> xr(xf.size());
    for (size_t i = 0; i < xf.size(); ++i) xr[i] = PrecisionType<f16>::to_f32(PrecisionType<f16>::from_f32(xf[i]));
    const Tensor2D<float> x32 = Tensor2D<float>::from_cpu_vector(ctx, xr, {batch, K});
    write_f32(dir + "/out32_fwd.bin", host_f32(ctx, back.forward(ctx, x32, batch, false, 2)));
    std::printf("convert round trip done\n");
    return 0;
}

}  // namespace

int main(int argc, char **argv) {
    if (argc < 2) return usage();
    const std::string cmd = argv[1];
    try {
        if (cmd == "selftest") return selftest();
        if (cmd == "chacha" && argc == 6)
            return chacha(std::atoi(argv[2]), argv[3], std::strtoull(argv[4], nullptr, 10), std::atoi(argv[5]));
        if (cmd == "pcg32" && argc == 5)
            return pcg32(std::strtoull(argv[2], nullptr, 10), std::strtoull(argv[3], nullptr, 10), std::atoi(argv[4]));
        if (cmd == "init" && argc == 8)
            return init_dump(argv[2], std::strtoull(argv[3], nullptr, 10), std::strtof(argv[4], nullptr),
                             std::strtoul(argv[5], nullptr, 10), std::strtoul(argv[6], nullptr, 10),
                             std::strtoul(argv[7], nullptr, 10));
        if (cmd == "ids") return ids();
        if (cmd == "st-demo" && argc == 3) return st_demo(argv[2]);
        if (cmd == "st-dump" && argc == 3) return st_dump(argv[2]);
        if (cmd == "sched" && argc >= 3) return sched(argc, argv);
        if (cmd == "convert" && argc == 7)
            return convert(argv[2], std::strtoul(argv[3], nullptr, 10), std::strtoul(argv[4], nullptr, 10),
                           std::strtoul(argv[5], nullptr, 10), std::strtoull(argv[6], nullptr, 10));
        if (cmd == "train" && argc == 3) {
            const auto spec = read_spec(std::string(argv[2]) + "/spec.txt");
            return spec.at("dtype") == "f16" ? train<f16>(argv[2], spec) : train<float>(argv[2], spec);
        }
    } catch (const Error &e) {
        std::fprintf(stderr, "soklyn error (status %d): %s\n", e.status(), e.what());
        return 3;
    } catch (const std::exception &e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 4;
    }
    return usage();
}
