// Task-2 driver: the VGG16-CIFAR10 main() of the reference (T2V:289-420) on
// the MI355X engine.  Reads the reference's assets -- the weights blob and
// the flat CIFAR-10 test set ({i}.bin = 3072 float32 in HWC order,
// label_onehot = N x 10 float32) -- and runs batches of B images through
// encode -> 13 same-padded 3x3 convolutions with a 2x2 min pool after conv
// 2, 4, 7, 10 and 13 (the VGG-16 plan, T2V:344-378) -> spiking FC layers ->
// a membrane-potential readout for the last FC layer (T2V:386) -> argmax,
// printing the reference's per-batch and summary lines.
//
//   vdttfs_vgg [--weights exported_models/snn_weights_vgg.bin]
//              [--data dataset_downloaded/cifar10_float/] [--n 10000] [--batch 1000]
//              [--T 80] [--tfs 40] [--delta 8] [--encode log|linear] [--tc-in 34.750164]
//              [--dropin] [--reps 1]
//
// Default: the whole layer loop is one vdttfs_net_forward per batch (LUTs
// resident, no host synchronisation inside the forward).  --dropin instead
// runs T2V's batch loop call for call on the drop-in entry points (the
// switch a maintainer makes in the reference program): per batch one H2D
// of the images, encode + synchronise, and per weighted layer
// vdttfs_update_luts (host expf, blocking upload) followed by
// vdttfs_launch_layer_sync / vdttfs_launch_fc_vmem_sync, pools through
// vdttfs_launch_pool_sync, then a D2H of the logits and the host argmax
// (T2V:337-402).  It also prints each layer's host time (LAYER_MS lines).
// --reps R repeats the whole inference R times and prints each run's time.
#include "driver_util.h"

namespace {

struct DropinLayerTime {
    double lut_s = 0, launch_s = 0;
};

// T2V:337-402 on the C ABI.  L: the topology built from the blob (pools
// inserted), dev: the blob's layers on the device (vdttfs_load_weights).
int run_dropin(vdttfs_ctx* ctx, const vdttfs_consts& c, const std::vector<vdttfs_layer_desc>& L,
               const vdttfs_dev_layer* dev, int n_dev, bool linear, float tc_in, float td_in,
               const std::vector<float>& imgs, const std::vector<float>& labels, int N, int B, int n_cls,
               int rep, std::vector<DropinLayerTime>& lt) {
    const int n_batches = (N + B - 1) / B;
    DevBuf d_img(ctx, (size_t)B * 3072 * 4), d_s0(ctx, (size_t)B * 3072 * 4);
    DevBuf d_decay(ctx, (size_t)(c.T + 1) * 4), d_th(ctx, (size_t)c.T * 4);
    std::vector<DevBuf*> outs;
    for (const vdttfs_layer_desc& d : L)
        outs.push_back(new DevBuf(ctx, (size_t)B * d.H_out * d.W_out * d.C_out * 4));
    std::vector<float> batch((size_t)B * 3072, 0.0f), h_out((size_t)B * n_cls);
    int total_correct = 0;
    using clk = std::chrono::steady_clock;
    std::cout << ">>> Starting Full " << N << " Inference (drop-in, call for call; " << n_batches
              << " batches of " << B << ")..." << std::endl;
    const auto t0 = clk::now();
    VD_CHECK(vdttfs_timer_begin(ctx));
    for (int bi = 0; bi < n_batches; ++bi) {
        const int s = bi * B, nb = std::min(B, N - s);
        std::copy(imgs.begin() + (size_t)s * 3072, imgs.begin() + (size_t)(s + nb) * 3072, batch.begin());
        VD_CHECK(vdttfs_h2d(ctx, d_img.p, batch.data(), batch.size() * 4));
        if (linear)
            VD_CHECK(vdttfs_encode_linear(ctx, d_img.as<float>(), d_s0.as<float>(), (int64_t)B * 3072));
        else
            VD_CHECK(vdttfs_encode_image(ctx, d_img.as<float>(), d_s0.as<float>(), (int64_t)B * 3072, tc_in,
                                         td_in));
        VD_CHECK(vdttfs_synchronize(ctx));
        const float* cur = d_s0.as<float>();
        float tc_i = tc_in, td_i = td_in;
        int wi = 0;
        for (size_t li = 0; li < L.size(); ++li) {
            const vdttfs_layer_desc& d = L[li];
            float* out = outs[li]->as<float>();
            if (d.kind == VDTTFS_LAYER_POOL) {
                const auto a = clk::now();
                VD_CHECK(vdttfs_launch_pool_sync(ctx, cur, out, d.H_in, d.W_in, d.C_in, B));
                lt[li].launch_s += seconds_since(a);
            } else {
                if (wi >= n_dev) {
                    std::cerr << "weights file has fewer layers than the topology" << std::endl;
                    return 1;
                }
                const vdttfs_dev_layer& w = dev[wi++];
                auto a = clk::now();
                VD_CHECK(vdttfs_update_luts(ctx, d_decay.as<float>(), d_th.as<float>(), tc_i, td_i, w.tc_fire,
                                            w.td));
                lt[li].lut_s += seconds_since(a);
                a = clk::now();
                if (d.kind == VDTTFS_LAYER_VMEM)
                    VD_CHECK(vdttfs_launch_fc_vmem_sync(ctx, cur, out, d.H_in * d.W_in * d.C_in, d.C_out,
                                                        w.d_kernel, w.d_bias, d_decay.as<float>(), B));
                else if (d.kind == VDTTFS_LAYER_FC)
                    VD_CHECK(vdttfs_launch_layer_sync(ctx, cur, out, 1, 1, d.H_in * d.W_in * d.C_in, 1, 1, d.C_out,
                                                      1, 1, w.td, w.d_kernel, w.d_bias, d_decay.as<float>(),
                                                      d_th.as<float>(), B, /*is_fc=*/1));
                else
                    VD_CHECK(vdttfs_launch_layer_sync(ctx, cur, out, d.H_in, d.W_in, d.C_in, d.H_out, d.W_out,
                                                      d.C_out, d.K_h, d.K_w, w.td, w.d_kernel, w.d_bias,
                                                      d_decay.as<float>(), d_th.as<float>(), B, /*is_fc=*/0));
                lt[li].launch_s += seconds_since(a);
                tc_i = w.tc_fire;
                td_i = w.td;
            }
            cur = out;
        }
        VD_CHECK(vdttfs_d2h(ctx, h_out.data(), cur, h_out.size() * 4));
        int bc = 0;
        for (int k = 0; k < nb; ++k) {  // T2V:389-396: strict > from -1e9
            float mv = -1e9f;
            int pc = -1;
            for (int i = 0; i < n_cls; ++i)
                if (h_out[(size_t)k * n_cls + i] > mv) {
                    mv = h_out[(size_t)k * n_cls + i];
                    pc = i;
                }
            if (pc == onehot_class(&labels[(size_t)(s + k) * n_cls], n_cls)) ++bc;
        }
        total_correct += bc;
        std::cout << "  -> Batch [" << bi + 1 << "/" << n_batches << "] Correct: " << bc << " / " << nb
                  << std::endl;
    }
    double ms = 0;
    VD_CHECK(vdttfs_timer_end(ctx, &ms));
    const double wall = seconds_since(t0);
    for (DevBuf* b : outs) delete b;
    std::cout << "\n=======================================" << std::endl;
    std::cout << "TIME-SORTED INPUT-GEN EARLY-EXIT COMPLETED (drop-in, run " << rep + 1 << ")" << std::endl;
    std::cout << "Total Images Processed: " << N << std::endl;
    std::cout << "Final Accuracy:         " << (float)total_correct / N * 100.0f << "%" << std::endl;
    std::cout << "Total Inference Time:   " << ms / 1000.0 << " seconds" << std::endl;
    std::cout << "Throughput:             " << N / (ms / 1000.0) << " images/sec" << std::endl;
    std::cout << "Host wall time:         " << wall << " seconds" << std::endl;
    std::cout << "=======================================" << std::endl;
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    const Args a(argc, argv);
    const int N = a.i("n", 10000);
    const int B = a.i("batch", 1000);
    const std::string weights = a.s("weights", "exported_models/snn_weights_vgg.bin");
    std::string dir = a.s("data", "dataset_downloaded/cifar10_float/");
    if (!dir.empty() && dir.back() != '/') dir += '/';
    if (N <= 0 || B <= 0) {
        std::cerr << "--n and --batch must be positive" << std::endl;
        return 2;
    }
    const vdttfs_consts c = {a.i("T", 80), a.f("tfs", 40.0f), a.i("delta", 8), 1.0f,
                             /*alpha_by_time=*/1, /*conv_same_pad=*/1};
    const bool linear = a.s("encode", "log") == "linear";
    const float tc_in = a.f("tc-in", 34.75016403198242f), td_in = a.f("td-in", 0.0f);

    std::cout << ">>> Loading VGG16 Weights..." << std::endl;
    vdttfs_blob* blob = nullptr;
    VD_CHECK(vdttfs_blob_read(weights.c_str(), &blob));
    std::vector<vdttfs_layer_desc> L;
    int H = 32, W = 32, C = 3, n_conv = 0, n_fc_total = 0;
    for (int i = 0; i < blob->num_layers; ++i) n_fc_total += blob->layers[i].ndim == 2;
    int n_fc = 0;
    for (int i = 0; i < blob->num_layers; ++i) {
        const vdttfs_blob_layer& b = blob->layers[i];
        vdttfs_layer_desc d{};
        d.kernel = b.kernel;
        d.bias = b.bias;
        d.tc_fire = b.tc_fire;
        d.td = b.td;
        if (b.ndim == 4) {
            if (b.c_in != C || b.k_h != 3 || b.k_w != 3) {
                std::cerr << "layer " << i << ": expected a 3x3 conv on " << C << " channels" << std::endl;
                return 1;
            }
            d.kind = VDTTFS_LAYER_CONV;
            d.H_in = d.H_out = H, d.W_in = d.W_out = W, d.C_in = C, d.C_out = b.c_out;
            d.K_h = d.K_w = 3;
            L.push_back(d);
            C = b.c_out;
            ++n_conv;
            if (n_conv == 2 || n_conv == 4 || n_conv == 7 || n_conv == 10 || n_conv == 13) {
                vdttfs_layer_desc p{};
                p.kind = VDTTFS_LAYER_POOL;
                p.H_in = H, p.W_in = W, p.C_in = C;
                p.H_out = H / 2, p.W_out = W / 2, p.C_out = C;
                L.push_back(p);
                H /= 2, W /= 2;
            }
        } else {
            if (b.c_in != H * W * C) {
                std::cerr << "layer " << i << ": FC takes " << b.c_in << " inputs, previous gives "
                          << H * W * C << std::endl;
                return 1;
            }
            ++n_fc;
            d.kind = n_fc == n_fc_total ? VDTTFS_LAYER_VMEM : VDTTFS_LAYER_FC;
            d.H_in = H, d.W_in = W, d.C_in = C;
            d.H_out = d.W_out = 1, d.C_out = b.c_out;
            d.K_h = d.K_w = 1;
            L.push_back(d);
            H = W = 1, C = b.c_out;
        }
    }
    const int n_cls = C;

    std::cout << ">>> Loading All " << N << " CIFAR-10 Test Images..." << std::endl;
    std::vector<float> imgs((size_t)N * 3072), labels((size_t)N * n_cls);
    for (int i = 0; i < N; ++i) read_exact(dir + std::to_string(i) + ".bin", &imgs[(size_t)i * 3072], 3072);
    read_exact(dir + "label_onehot", labels.data(), labels.size());

    vdttfs_ctx* ctx = nullptr;
    VD_CHECK(vdttfs_create(&c, 0, &ctx));
    const int reps = std::max(1, a.i("reps", 1));
    if (a.s("dropin", "0") == "1") {
        vdttfs_blob_free(blob);
        vdttfs_dev_layer* dev = nullptr;
        int n_dev = 0;
        VD_CHECK(vdttfs_load_weights(ctx, weights.c_str(), &dev, &n_dev));
        std::vector<DropinLayerTime> lt(L.size());
        for (int r = 0; r < reps; ++r) {
            if (r == reps - 1) lt.assign(L.size(), DropinLayerTime{});  // per-layer times of the last run
            const int rc = run_dropin(ctx, c, L, dev, n_dev, linear, tc_in, td_in, imgs, labels, N, B, n_cls, r, lt);
            if (rc) return rc;
        }
        static const char* kinds[] = {"conv", "fc", "pool", "vmem"};
        for (size_t li = 0; li < L.size(); ++li)
            std::cout << "LAYER_MS i=" << li << " kind=" << kinds[L[li].kind] << " lut_ms=" << lt[li].lut_s * 1e3
                      << " launch_ms=" << lt[li].launch_s * 1e3 << std::endl;
        VD_CHECK(vdttfs_free_weights(ctx, dev, n_dev));
        vdttfs_destroy(ctx);
        return 0;
    }
    vdttfs_net* net = nullptr;
    VD_CHECK(vdttfs_net_create(ctx, L.data(), (int)L.size(), B, 3072,
                               linear ? VDTTFS_ENCODE_LINEAR : VDTTFS_ENCODE_LOG, tc_in, td_in,
                               VDTTFS_READOUT_ARGMAX, &net));
    vdttfs_blob_free(blob);
    const int n_batches = (N + B - 1) / B;
    std::vector<int32_t> pred((size_t)B);
    std::vector<float> batch((size_t)B * 3072, 0.0f);
    int total_correct = 0;
    {
        DevBuf d_img(ctx, batch.size() * 4), d_pred(ctx, pred.size() * 4);
        std::cout << ">>> Starting Full " << N << " Inference (time-sorted input-gen early-exit, "
                  << n_batches << " batches of " << B << ")..." << std::endl;
        const auto t0 = std::chrono::steady_clock::now();
        VD_CHECK(vdttfs_timer_begin(ctx));
        for (int bi = 0; bi < n_batches; ++bi) {
            const int s = bi * B, nb = std::min(B, N - s);
            std::copy(imgs.begin() + (size_t)s * 3072, imgs.begin() + (size_t)(s + nb) * 3072, batch.begin());
            VD_CHECK(vdttfs_h2d(ctx, d_img.p, batch.data(), batch.size() * 4));
            VD_CHECK(vdttfs_net_forward(net, d_img.as<float>(), d_pred.as<int32_t>()));
            VD_CHECK(vdttfs_d2h(ctx, pred.data(), d_pred.p, pred.size() * 4));
            int bc = 0;
            for (int k = 0; k < nb; ++k)
                if (pred[k] == onehot_class(&labels[(size_t)(s + k) * n_cls], n_cls)) ++bc;
            total_correct += bc;
            std::cout << "  -> Batch [" << bi + 1 << "/" << n_batches << "] Correct: " << bc << " / " << nb
                      << std::endl;
        }
        double ms = 0;
        VD_CHECK(vdttfs_timer_end(ctx, &ms));
        const double wall = seconds_since(t0);
        std::cout << "\n=======================================" << std::endl;
        std::cout << "TIME-SORTED INPUT-GEN EARLY-EXIT COMPLETED" << std::endl;
        std::cout << "Total Images Processed: " << N << std::endl;
        std::cout << "Final Accuracy:         " << (float)total_correct / N * 100.0f << "%" << std::endl;
        std::cout << "Total Inference Time:   " << ms / 1000.0 << " seconds" << std::endl;
        std::cout << "Throughput:             " << N / (ms / 1000.0) << " images/sec" << std::endl;
        std::cout << "Host wall time:         " << wall << " seconds" << std::endl;
        std::cout << "=======================================" << std::endl;
    }
    vdttfs_net_destroy(net);
    vdttfs_destroy(ctx);
    return 0;
}
