// cli.cpp - `scunet`, the command-line denoiser over libscunet_hip.so.
//
// The reference's src/main.rs with its `--device gpu` path: the same flags, messages and
// exit codes (2 for a usage error or a refused request, 1 for a failure), PNG in and PNG
// out through scunet_image_read / scunet_image_write (src/image.rs), and the forward
// through scunet_hip_run (backend::run: replicate pad, forward, crop; here on the device).
//
// This build is the MI355X backend only. The reference's CPU backend is not part of it,
// so `--device cpu` is refused the way a reference build without its GPU feature refuses
// `--device gpu` (main.rs:183-187), and a device that cannot be brought up is an error
// whether or not the GPU was named (the reference falls back to its CPU backend when it
// was not, main.rs:176-182).
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "../../include/scunet_hip.h"
#include "../../include/scunet_image.h"

namespace {

const char* kVersion = "0.1.0";

[[noreturn]] void usage() {
    std::fprintf(stderr,
                 "scunet %s - SCUNet real-world image denoising on MI355X (HIP)\n"
                 "\n"
                 "USAGE:\n"
                 "    scunet -m <weights.safetensors> -i <in.png> -o <out.png> [options]\n"
                 "\n"
                 "OPTIONS:\n"
                 "    -m, --model <path>    converted .safetensors checkpoint (python -m scunet_hip.convert)\n"
                 "    -i, --input <path>    input PNG, 8-bit, RGB or grayscale\n"
                 "    -o, --output <path>   where to write the denoised PNG\n"
                 "        --device <dev>    gpu (the default; `cuda` and `hip` are accepted for gpu)\n"
                 "        --gpu             same as --device gpu\n"
                 "        --fp16            fp16 matrix-core operands with fp32 accumulation\n"
                 "                          (faster; within 4e-3 of the fp32 result)\n"
                 "    -q, --quiet           no progress output\n"
                 "    -h, --help            this text\n"
                 "    -V, --version         print the version\n"
                 "\n"
                 "The model takes the image at its native resolution - there is no tile size to\n"
                 "choose and no `--tile` flag.\n",
                 kVersion);
    std::exit(2);
}

struct Args {
    std::string weights, input, output, device = "gpu";
    bool fp16 = false, quiet = false;
};

Args parse(int argc, char** argv) {
    Args a;
    bool have_w = false, have_i = false, have_o = false;
    for (int k = 1; k < argc; ++k) {
        std::string s = argv[k];
        auto take = [&](const char* what) -> std::string {
            if (k + 1 >= argc) {
                std::fprintf(stderr, "scunet: %s needs a value\n", what);
                usage();
            }
            return argv[++k];
        };
        if (s == "-m" || s == "--model" || s == "--weights") {
            a.weights = take("--model");
            have_w = true;
        } else if (s == "-i" || s == "--input" || s == "--in") {
            a.input = take("--input");
            have_i = true;
        } else if (s == "-o" || s == "--output" || s == "--out") {
            a.output = take("--output");
            have_o = true;
        } else if (s == "--device") {
            a.device = take("--device");
        } else if (s == "--cpu") {
            a.device = "cpu";
        } else if (s == "--gpu") {
            a.device = "gpu";
        } else if (s == "--fp16") {
            a.fp16 = true;
        } else if (s == "-q" || s == "--quiet") {
            a.quiet = true;
        } else if (s == "-h" || s == "--help") {
            usage();
        } else if (s == "-V" || s == "--version") {
            std::printf("scunet %s\n", kVersion);
            std::exit(0);
        } else if (s == "--tile" || s == "--tile-pad") {
            // main.rs:96-105: answered with the reason, never silently accepted.
            std::fprintf(stderr, "scunet: `%s` is not supported: this engine runs a whole image at once\n", s.c_str());
            std::fprintf(stderr, "scunet: (SCUNet pads by replication to a multiple of 64 and has no tile geometry)\n");
            std::exit(2);
        } else {
            std::fprintf(stderr, "scunet: unknown argument `%s`\n", s.c_str());
            usage();
        }
    }
    if (!have_w) {
        std::fprintf(stderr, "scunet: --model is required (see python -m scunet_hip.convert)\n");
        usage();
    }
    if (!have_i || !have_o) {
        std::fprintf(stderr, "scunet: --input and --output are required\n");
        usage();
    }
    return a;
}

}  // namespace

int main(int argc, char** argv) {
    Args a = parse(argc, argv);
    if (a.device == "cpu") {
        std::fprintf(stderr, "scunet: this build is the HIP backend only and has no cpu device; use --device gpu\n");
        return 2;
    }
    if (a.device != "gpu" && a.device != "cuda" && a.device != "hip") {
        std::fprintf(stderr, "scunet: unknown device `%s` (gpu or cpu)\n", a.device.c_str());
        return 2;
    }

    scunet_hip* h = nullptr;
    if (scunet_hip_create(a.weights.c_str(), &h) != 0) {
        std::fprintf(stderr, "scunet: %s\n", scunet_hip_create_error());
        return 1;
    }
    int in_nc = 0, dim = 0, head_dim = 0, window = 0, config[7];
    scunet_hip_arch(h, &in_nc, &dim, &head_dim, &window, config);
    if (!a.quiet)
        std::fprintf(stderr, "scunet %s: %s (%s in_nc %d, dim %d, window %d)\n", kVersion, scunet_hip_variant(h),
                     a.weights.c_str(), in_nc, dim, window);

    float* x = nullptr;
    size_t c = 0, hh = 0, ww = 0;
    if (scunet_image_read(a.input.c_str(), &x, &c, &hh, &ww) != 0) {
        std::fprintf(stderr, "scunet: %s\n", scunet_image_error());
        scunet_hip_destroy(h);
        return 1;
    }
    if (int(c) != in_nc) {
        std::fprintf(stderr, "scunet: %s: %zu channels, but this checkpoint takes %d (a %s model)\n",
                     a.input.c_str(), c, in_nc, scunet_hip_variant(h));
        scunet_image_free(x);
        scunet_hip_destroy(h);
        return 2;
    }
    if (a.fp16 && scunet_hip_set_precision(h, SCUNET_HIP_FP16) != 0) {
        std::fprintf(stderr, "scunet: %s\n", scunet_hip_last_error(h));
        scunet_image_free(x);
        scunet_hip_destroy(h);
        return 1;
    }
    if (!a.quiet) std::fprintf(stderr, "scunet: device hip%s\n", a.fp16 ? " (fp16 operands)" : "");

    auto t0 = std::chrono::steady_clock::now();
    std::vector<float> y;
    try {
        y.resize(c * hh * ww);
    } catch (const std::bad_alloc&) {
        std::fprintf(stderr, "scunet: out of host memory for a %zux%zu image\n", ww, hh);
        scunet_image_free(x);
        scunet_hip_destroy(h);
        return 1;
    }
    int rc = scunet_hip_run(h, x, c, hh, ww, y.data());
    scunet_image_free(x);
    if (rc != 0) {
        std::fprintf(stderr, "scunet: %s\n", scunet_hip_last_error(h));
        scunet_hip_destroy(h);
        return 1;
    }
    double dt = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    scunet_hip_destroy(h);
    if (!a.quiet) std::fprintf(stderr, "scunet: %zux%zu -> %zux%zu in %.2fs\n", ww, hh, ww, hh, dt);
    if (scunet_image_write(a.output.c_str(), y.data(), c, hh, ww) != 0) {
        std::fprintf(stderr, "scunet: %s\n", scunet_image_error());
        return 1;
    }
    return 0;
}
