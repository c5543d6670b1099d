// The rocm GEMM kernels' tunable settings (TunableKernel "matmul", "gemm" and
// "gemm_strided_batched", as the reference's tuner sees them: src/core/dispatcher.hpp:226-239):
// registration, key, defaults, the search space and `allowed`, and every allowed point of the
// space run through the kernel the way the tuner runs it (args.tuning set), each bit-exact on
// quarter-integer inputs, whose products sum exactly in any order (split-K included). Without a
// rocm device there is nothing registered to check.
#include "core/dispatcher.hpp"
#include "core/registry.hpp"
#include "core/tuning.hpp"
#include "mensurflow/mensurflow.hpp"
#include "mensurflow/tuning.hpp"
#include "oracle_cpu.hpp"
#include "test_util.hpp"

#include "mfr_rocm.h"

#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

using namespace mensurflow;
using namespace mensurflow::detail;

namespace {

// C = alpha * A B + beta * C0 + bias, in double (exact for quarter-integer inputs), as float.
std::vector<float> exact_gemm(const std::vector<float>& a, const std::vector<float>& b,
                              std::int64_t m, std::int64_t n, std::int64_t k, double alpha,
                              const std::vector<float>* c0, double beta,
                              const std::vector<float>* bias) {
    std::vector<float> out(static_cast<std::size_t>(m * n));
    for (std::int64_t i = 0; i < m; ++i) {
        for (std::int64_t j = 0; j < n; ++j) {
            double sum = 0.0;
            for (std::int64_t p = 0; p < k; ++p) {
                sum += static_cast<double>(a[static_cast<std::size_t>(i * k + p)]) *
                       b[static_cast<std::size_t>(p * n + j)];
            }
            double v = alpha * sum;
            if (c0 != nullptr) {
                v += beta * (*c0)[static_cast<std::size_t>(i * n + j)];
            }
            if (bias != nullptr) {
                v += (*bias)[static_cast<std::size_t>(j)];
            }
            out[static_cast<std::size_t>(i * n + j)] = static_cast<float>(v);
        }
    }
    return out;
}

TuningConfig point(std::int64_t tile, std::int64_t stage, std::int64_t splits) {
    TuningConfig c;
    c.values[0] = tile;
    c.values[1] = stage;
    c.values[2] = splits;
    c.size = 3;
    return c;
}

// Depth ranges mfr_sgemm runs when `splits` are asked for at depth k: ranges a multiple of 32
// deep, so fewer when the depth is short.
std::int64_t ranges_run(std::int64_t k, std::int64_t splits) {
    const std::int64_t per = ((k + splits - 1) / splits + 31) / 32 * 32;
    return splits == 1 ? 1 : (k + per - 1) / per;
}

// Runs every point of `op`'s space that `allowed` accepts and checks the output each time.
// Points refused are exactly the thin path (no product here is thin), the panel path where the
// product does not fit it (panel: it does, and then only unsplit), and split counts the depth k
// is too short for; with staging off, the 256x256 tile reads an operand 16-byte loads cannot read
// (the matmul and batched cases) in place.
void sweep(Device device, OpId op, OpArgs args, const std::vector<float>& want, std::int64_t k,
           const std::string& what, bool panel = false) {
    Registry& registry = Registry::instance();
    const TunableKernel& tunable = *registry.dispatcher().tunable({op, DeviceType::ROCm, DType::F32});
    const KernelFn kernel = registry.dispatcher().lookup({op, DeviceType::ROCm, DType::F32});
    Stream& stream = registry.get(device).stream(device.index);
    const std::vector<SearchRegion> regions = tunable.space(args);
    test::require(regions.size() == 1 && regions[0].axes.size() == 3, what + ": one region");
    const SearchRegion& region = regions[0];
    test::require(region.start.size == 3 && region.start.values[0] > MFR_TILE_AUTO &&
                      region.start.values[0] < MFR_TILE_COUNT && region.start.values[2] >= 1,
                  what + ": the start is a fixed tile and split count");
    test::require(tunable.allowed(args, region.start), what + ": the start is allowed");
    int ran = 0, counts = 0;
    for (std::int64_t splits : region.axes[2].values) {
        counts += ranges_run(k, splits) == splits;
        for (std::int64_t tile : region.axes[0].values) {
            for (std::int64_t stage : region.axes[1].values) {
                const TuningConfig config = point(tile, stage, splits);
                const bool allowed = tunable.allowed(args, config);
                // None of these products is thin enough (m, n > 8) for the thin path.
                const bool expected =
                    tile != MFR_TILE_THIN && ranges_run(k, splits) == splits &&
                    (tile != MFR_TILE_PANEL || (panel && splits == 1));
                const std::string name = "tile " + std::to_string(tile) + " stage " +
                                         std::to_string(stage) + " splits " +
                                         std::to_string(splits);
                test::require(allowed == expected, what + ": allowed(" + name + ")");
                if (!allowed) {
                    continue;
                }
                args.tuning = config;
                kernel(args, stream);
                test::require(test::same_bits(args.outputs[0].to_vector<float>(), want),
                              what + ": " + name);
                ++ran;
            }
        }
    }
    test::require(counts >= 2 && ran == 10 * counts + (panel ? 2 : 0),
                  what + ": every allowed point ran");
    // Not a point: AUTO is only the default, and unknown values are refused.
    test::require(!tunable.allowed(args, point(MFR_TILE_AUTO, MFR_STAGE_NEVER, 1)) &&
                      !tunable.allowed(args, point(MFR_TILE_64x64, 7, 1)) &&
                      !tunable.allowed(args, point(MFR_TILE_64x64, MFR_STAGE_NEVER, 0)) &&
                      !tunable.allowed(args, point(MFR_TILE_64x64, MFR_STAGE_NEVER, 65)),
                  what + ": invalid points refused");
}

void test_registration() {
    const Dispatcher& dispatcher = Registry::instance().dispatcher();
    const std::pair<OpId, const char*> ops[] = {
        {OpId::Matmul, "matmul"}, {OpId::Gemm, "gemm"}, {OpId::GemmBatched, "gemm_strided_batched"}};
    for (const auto& [op, name] : ops) {
        const TunableKernel* t = dispatcher.tunable({op, DeviceType::ROCm, DType::F32});
        test::require(t != nullptr && t->name == name, std::string(name) + " is tunable on rocm");
        test::require(t->params == std::vector<std::string>{"tile", "stage", "splits"}, "params");
        const TuningConfig d = t->defaults();
        test::require(d.size == 3 && d.values[0] == MFR_TILE_AUTO &&
                          d.values[1] == MFR_STAGE_AUTO && d.values[2] == 0,
                      "defaults leave every setting to the kernel");
    }
}

void test_matmul(Device device) {
    const std::int64_t m = 300, n = 261, k = 1023; // odd k and n: 4-byte loads in place
    const auto av = test::quarter_input(m * k, 61);
    const auto bv = test::quarter_input(k * n, 62);
    OpArgs args;
    args.inputs = {Tensor::from_vector(av, {m, k}, device), Tensor::from_vector(bv, {k, n}, device)};
    args.outputs = {Tensor::empty({m, n}, DType::F32, device)};
    const TunableKernel& t =
        *Registry::instance().dispatcher().tunable({OpId::Matmul, DeviceType::ROCm, DType::F32});
    test::require(t.key(args) == std::vector<std::int64_t>{m, n, k}, "matmul key");
    const auto want = exact_gemm(av, bv, m, n, k, 1.0, nullptr, 0.0, nullptr);
    sweep(device, OpId::Matmul, args, want, k, "matmul 300x261x1023");
}

void test_gemm_fused(Device device) {
    // B stored [n, k] and read transposed, as configs[2]; alpha, beta*C0 and a bias.
    const std::int64_t m = 257, n = 200, k = 96; // aligned: every point runs
    const auto av = test::quarter_input(m * k, 63);
    const auto bt = test::quarter_input(n * k, 64);
    const auto cv = test::quarter_input(m * n, 65);
    const auto biasv = test::quarter_input(n, 66);
    std::vector<float> bv(static_cast<std::size_t>(k * n));
    for (std::int64_t p = 0; p < k; ++p) {
        for (std::int64_t j = 0; j < n; ++j) {
            bv[static_cast<std::size_t>(p * n + j)] = bt[static_cast<std::size_t>(j * k + p)];
        }
    }
    OpArgs args;
    args.inputs = {Tensor::from_vector(av, {m, k}, device),
                   Tensor::from_vector(bt, {n, k}, device).transpose(0, 1),
                   Tensor::from_vector(cv, {m, n}, device), Tensor::from_vector(biasv, {n}, device)};
    args.outputs = {Tensor::empty({m, n}, DType::F32, device)};
    args.alpha = 1.5f;
    args.beta = 0.5f;
    args.has_bias = true;
    const auto want = exact_gemm(av, bv, m, n, k, 1.5, &cv, 0.5, &biasv);
    sweep(device, OpId::Gemm, args, want, k, "gemm 257x200x96 NT");
}

void test_batched(Device device) {
    // [2, 3] batch, B shared over the first dimension (stride 0), odd k.
    const std::int64_t bs = 2, h = 3, m = 70, n = 45, k = 63;
    const auto av = test::quarter_input(bs * h * m * k, 67);
    const auto bv = test::quarter_input(h * k * n, 68);
    OpArgs args;
    args.inputs = {Tensor::from_vector(av, {bs, h, m, k}, device),
                   Tensor::from_vector(bv, {1, h, k, n}, device).expand({bs, h, k, n})};
    args.outputs = {Tensor::empty({bs, h, m, n}, DType::F32, device)};
    args.alpha = 0.5f;
    args.beta = 0.0f;
    const TunableKernel& t = *Registry::instance().dispatcher().tunable(
        {OpId::GemmBatched, DeviceType::ROCm, DType::F32});
    test::require(t.key(args) == std::vector<std::int64_t>{bs * h, m, n, k}, "batched key");
    std::vector<float> want;
    for (std::int64_t i = 0; i < bs; ++i) {
        for (std::int64_t j = 0; j < h; ++j) {
            const auto off_a = static_cast<std::ptrdiff_t>((i * h + j) * m * k);
            const auto off_b = static_cast<std::ptrdiff_t>(j * k * n);
            const std::vector<float> a(av.begin() + off_a, av.begin() + off_a + m * k);
            const std::vector<float> b(bv.begin() + off_b, bv.begin() + off_b + k * n);
            const auto c = exact_gemm(a, b, m, n, k, 0.5, nullptr, 0.0, nullptr);
            want.insert(want.end(), c.begin(), c.end());
        }
    }
    sweep(device, OpId::GemmBatched, args, want, k, "batched 2x3x70x45x63");
}

void test_batched_scores(Device device) {
    // Attention's scores q k^T: a short, aligned depth with both operands read along k, so the
    // panel path is a point of the space (unsplit only).
    const std::int64_t bs = 3, m = 300, n = 130, k = 64;
    const auto qv = test::quarter_input(bs * m * k, 69);
    const auto kv = test::quarter_input(bs * n * k, 70);
    OpArgs args;
    args.inputs = {Tensor::from_vector(qv, {bs, m, k}, device),
                   Tensor::from_vector(kv, {bs, n, k}, device).transpose(1, 2)};
    args.outputs = {Tensor::empty({bs, m, n}, DType::F32, device)};
    args.alpha = 0.125f;
    args.beta = 0.0f;
    std::vector<float> want;
    for (std::int64_t i = 0; i < bs; ++i) {
        const std::vector<float> a(qv.begin() + static_cast<std::ptrdiff_t>(i * m * k),
                                   qv.begin() + static_cast<std::ptrdiff_t>((i + 1) * m * k));
        std::vector<float> b(static_cast<std::size_t>(k * n));
        for (std::int64_t p = 0; p < k; ++p) {
            for (std::int64_t j = 0; j < n; ++j) {
                b[static_cast<std::size_t>(p * n + j)] =
                    kv[static_cast<std::size_t>((i * n + j) * k + p)];
            }
        }
        const auto c = exact_gemm(a, b, m, n, k, 0.125, nullptr, 0.0, nullptr);
        want.insert(want.end(), c.begin(), c.end());
    }
    sweep(device, OpId::GemmBatched, args, want, k, "batched scores 3x300x130x64", true);
}

void test_start_is_the_automatic_choice(Device device) {
    // configs[3]'s shape: large and misaligned, so AUTO stages both operands.
    const std::int64_t m = 2045, n = 2051, k = 1023;
    OpArgs args;
    args.inputs = {Tensor::zeros({m, k}, DType::F32, device), Tensor::zeros({k, n}, DType::F32, device)};
    args.outputs = {Tensor::empty({m, n}, DType::F32, device)};
    const TunableKernel& t =
        *Registry::instance().dispatcher().tunable({OpId::Matmul, DeviceType::ROCm, DType::F32});
    const auto regions = t.space(args);
    test::require(regions.size() == 1 && regions[0].start.values[1] == MFR_STAGE_ALWAYS,
                  "a large misaligned product starts staged");
    // Nothing to compute: nothing to tune.
    OpArgs empty;
    empty.inputs = {Tensor::zeros({0, k}, DType::F32, device), Tensor::zeros({k, n}, DType::F32, device)};
    empty.outputs = {Tensor::empty({0, n}, DType::F32, device)};
    test::require(t.space(empty).empty(), "an empty product has no space");
}

// ---- tuned placement: the results file and dispatch()'s hook ------------------------------------

std::string results_path(const char* name) {
    if (const char* dir = std::getenv("MFR_TUNING_DIR")) {
        return std::string(dir) + "/" + name;
    }
    return std::string("/tmp/") + name;
}

void test_results_file_round_trip() {
    TuningCache cache;
    TuningEntry kernel{"Some CPU | gfx950", "matmul", "rocm", 2, "m=300 n=200 k=500",
                       {{"tile", 5}, {"stage", 1}, {"splits", 2}}, 0.0123, 0.0456, "tested"};
    TuningEntry place{"Some CPU | gfx950", "matmul", "auto", 1, "data=cpu f32 300x500 500x200",
                      {{"gpu", 1}}, 0.5, 12.25, "tested"};
    cache.store(kernel);
    cache.store(place);
    const std::string path = results_path("mfr_tuning_round_trip.txt");
    cache.save(path);
    TuningCache back;
    back.load(path);
    test::require(back.entries().size() == 2, "two results read back");
    const TuningEntry* k = back.find(kernel.machine, "matmul", "rocm", 2, kernel.key);
    test::require(k != nullptr && k->config == kernel.config && k->mode == "tested" &&
                      std::abs(k->best_ms - 0.0123) < 1e-9,
                  "the kernel line reads back");
    test::require(back.find(kernel.machine, "matmul", "rocm", 1, kernel.key) == nullptr,
                  "another version does not match");
    test::require(back.find(place.machine, "matmul", "auto", 1, place.key) != nullptr,
                  "the device-choice line reads back");
    // The reference's own line shape, written by hand (extra spaces are allowed in the key).
    {
        std::ofstream out(path);
        out << "# mensurflow tuning results\n\nmachine A | B\n"
            << "matmul  metal v1  m=64   n=256 k=784 -> kernel=1 bm=32 | 0.0410 ms (default "
               "0.0470 ms) tested\n";
    }
    back.load(path);
    test::require(back.entries().size() == 1 && back.entries()[0].key == "m=64 n=256 k=784" &&
                      back.entries()[0].device == "metal",
                  "a hand-written line is read");
    {
        std::ofstream out(path);
        out << "machine A\nmatmul rocm v2 m=1 -> tile=5 | 1 ms (default 2 ms) tested\n"
            << "matmul rocm v2 m=2 -> tile=x | 1 ms (default 2 ms) tested\n";
    }
    bool threw = false;
    try {
        back.load(path);
    } catch (const std::runtime_error& e) {
        threw = std::string(e.what()).find(":3: ") != std::string::npos;
    }
    test::require(threw, "a malformed line is reported with its number");
    // Each malformed form is reported with its line number and the part that did not match.
    const std::pair<const char*, const char*> malformed[] = {
        {"matmul rocm v2 m=1 -> tile=5 | 1 ms (default 2 ms) tested\n",
         ":1: a result before any 'machine' line"},
        {"machine A\nmatmul rocm v2 m=1 -> tile=5 1 ms (default 2 ms) tested\n",
         ":2: expected '<op> <device> v<version> <key> -> <settings> | "},
        {"machine A\nmatmul rocm 2 m=1 -> tile=5 | 1 ms (default 2 ms) tested\n",
         ":2: expected '<op> <device> v<version>' at the start"},
        {"machine A\n\n# note\nmatmul rocm v2 m=1 -> tile=5 | 1 ms tested\n",
         ":4: expected '<ms> ms (default <ms> ms) <mode>' after '|'"},
        {"machine A\nmatmul rocm v2 m=1 -> tile=99999999999999999999 | 1 ms (default 2 ms) t\n",
         ":2: number out of range: "},
    };
    for (const auto& [text, message] : malformed) {
        {
            std::ofstream out(path);
            out << text;
        }
        std::string what;
        try {
            back.load(path);
        } catch (const std::runtime_error& e) {
            what = e.what();
        }
        test::require(what.find(message) != std::string::npos,
                      std::string("malformed line reported as '") + message + "', got '" + what + "'");
    }
    // As lenient as the reference's reader: the version is the number 'v' starts ("v2x" is 2),
    // and words after the mode are ignored.
    {
        std::ofstream out(path);
        out << "machine A\nmatmul rocm v2x m=1 -> tile=5 | 1 ms (default 2 ms) tested by hand\n";
    }
    back.load(path);
    test::require(back.entries().size() == 1 && back.entries()[0].version == 2 &&
                      back.entries()[0].mode == "tested" && back.entries()[0].best_ms == 1.0,
                  "a version with a suffix and words after the mode are read");
    // Older "place" lines are skipped; empty settings and an empty key read back as empty.
    {
        std::ofstream out(path);
        out << "  machine  A | B  \nplace matmul 1x2 -> cpu\n"
            << "matmul rocm v2  ->  | 0.5 ms (default 0.5 ms) tested\n";
    }
    back.load(path);
    test::require(back.entries().size() == 1 && back.entries()[0].machine == "A | B" &&
                      back.entries()[0].key.empty() && back.entries()[0].config.empty() &&
                      back.entries()[0].best_ms == 0.5 && back.entries()[0].mode == "tested",
                  "place lines skipped, empty key and settings read");
    std::remove(path.c_str());
}

// An Auto matmul under a scope holding `cache`; returns the recorded calls and the result.
std::vector<RecordedCall> run_recorded(const TuningCache& cache, const Tensor& a, const Tensor& b,
                                       std::vector<float>* result) {
    std::vector<RecordedCall> calls;
    {
        const TuningScope scope({&cache, &calls});
        const Tensor c = matmul(a, b); // Execution::Auto
        *result = c.to_vector<float>();
    }
    return calls;
}

void test_auto_placement_on_cpu() {
    // A stored gpu=0 keeps an Auto call on the CPU, and no entry leaves it there too.
    const std::int64_t m = 20, n = 12, k = 33;
    const auto av = test::quarter_input(m * k, 71);
    const auto bv = test::quarter_input(k * n, 72);
    const Tensor a = Tensor::from_vector(av, {m, k});
    const Tensor b = Tensor::from_vector(bv, {k, n});
    OpArgs args{{a, b}, {}};
    TuningCache cache;
    cache.store({machine_name(), "matmul", kAutoDevice, 1, placement_key(args, a.device()),
                 {{"gpu", 0}}, 1.0, 1.0, "tested"});
    test::require(placement_key(args, a.device()) == "data=cpu f32 20x33 33x12",
                  "placement key as the reference writes it");
    std::vector<float> c;
    const auto calls = run_recorded(cache, a, b, &c);
    test::require(calls.size() == 1 && calls[0].op == OpId::Matmul &&
                      calls[0].execution == Execution::Auto &&
                      calls[0].device == Device{DeviceType::CPU, 0},
                  "gpu=0: the call runs on the CPU");
    test::require(test::same_bits(c, exact_gemm(av, bv, m, n, k, 1.0, nullptr, 0.0, nullptr)),
                  "the CPU result is exact");
}

void test_tuner_places_auto_on_rocm(Device device) {
    // configs[0]-like product on CPU data, called with Execution::Auto. The tuner times the CPU
    // against rocm:0 (copies included) and every allowed point of the rocm matmul's space, and
    // stores both; running under those results places the call on rocm:0 with the stored tile.
    const std::int64_t m = 512, n = 384, k = 1024;
    const auto av = test::quarter_input(m * k, 81);
    const auto bv = test::quarter_input(k * n, 82);
    const Tensor a = Tensor::from_vector(av, {m, k});
    const Tensor b = Tensor::from_vector(bv, {k, n});
    const auto want = exact_gemm(av, bv, m, n, k, 1.0, nullptr, 0.0, nullptr);
    const std::string path = results_path("mfr_tuning_results.txt");
    std::remove(path.c_str());
    Algorithm step([](const std::vector<Tensor>& in) {
        return std::vector<Tensor>{matmul(in[0], in[1])};
    });
    TuneOptions options;
    options.min_time_s = 0.005;
    Tuner tuner(path);
    const TuneReport report = tuner.tune(step, {a, b}, options);
    std::cout << tuner.describe();
    test::require(report.calls.size() == 2, "a device choice and a kernel result");

    TuningCache cache;
    cache.load(path);
    OpArgs args{{a, b}, {}};
    const TuningEntry* place = cache.find(machine_name(), "matmul", kAutoDevice, 1,
                                          placement_key(args, a.device()));
    test::require(place != nullptr && place->config == TuningValues{{"gpu", 1}},
                  "the GPU wins this product and is stored");
    const TunableKernel& tunable =
        *Registry::instance().dispatcher().tunable({OpId::Matmul, DeviceType::ROCm, DType::F32});
    OpArgs on_gpu{{a.to(device), b.to(device)}, {Tensor::empty({m, n}, DType::F32, device)}};
    const std::string key = call_key(tunable, on_gpu, device);
    test::require(key == "m=512 n=384 k=1024", "kernel key as the reference writes it");
    const TuningEntry* kernel = cache.find(machine_name(), "matmul", "rocm", tunable.version, key);
    test::require(kernel != nullptr && kernel->config.size() == 3, "the tile is stored");

    std::vector<float> c;
    const auto calls = run_recorded(cache, a, b, &c);
    test::require(calls.size() == 1 && calls[0].device == device, "the Auto call ran on rocm:0");
    test::require(test::same_bits(c, want), "bit-exact on quarter-integer inputs");
    // The hook, as dispatch() called it for that call (the record is taken before the settings
    // are applied): it picks rocm:0 and sets the stored tile.
    {
        OpArgs seen = calls[0].args;
        const TuningScope scope({&cache, nullptr});
        const Device target = apply_tuning(OpId::Matmul, Execution::Auto, a.device(), seen);
        test::require(target == device && seen.tuning == to_config(tunable, kernel->config) &&
                          seen.tuning.values[0] == kernel->config[0].second,
                      "the hook applies the stored settings");
    }
    // The settings reach the kernel: a stored thin tile, which this product cannot take, makes
    // the same call fail in the kernel.
    {
        TuningCache refused = cache;
        TuningEntry thin = *kernel;
        thin.config = {{"tile", MFR_TILE_THIN}, {"stage", MFR_STAGE_NEVER}, {"splits", 1}};
        refused.store(thin);
        bool kernel_refused = false;
        try {
            std::vector<float> unused;
            run_recorded(refused, a, b, &unused);
        } catch (const NotImplemented&) {
            kernel_refused = true;
        }
        test::require(kernel_refused, "a stored thin tile reaches mfr_sgemm, which refuses it");
    }
    // The public path: Algorithm::run with the tuner gives the same bits.
    const std::vector<Tensor> out = step.run({a, b}, tuner);
    test::require(out.size() == 1 && test::same_bits(out[0].to_vector<float>(), want),
                  "Algorithm::run(inputs, tuner)");
    std::cout << "  tuned: " << to_string(kernel->config) << " (" << kernel->best_ms
              << " ms, default " << kernel->default_ms << " ms)\n";
}

} // namespace

int main(int argc, char** argv) {
    return test::run("tuning_test", argc, argv, [] {
        test::register_oracle_cpu_kernels();
        test_results_file_round_trip();
        test_auto_placement_on_cpu();
        bool rocm = false;
        for (Device device : test::devices()) {
            if (device.type != DeviceType::ROCm) {
                continue;
            }
            rocm = true;
            std::cout << "  gemm tunables on " << to_string(device) << '\n';
            test_registration();
            test_matmul(device);
            test_gemm_fused(device);
            test_batched(device);
            test_batched_scores(device);
            test_start_is_the_automatic_choice(device);
            test_tuner_places_auto_on_rocm(device);
        }
        if (!rocm) {
            std::cout << "  no rocm device: the backend registers no tunables to check\n";
        }
    });
}
