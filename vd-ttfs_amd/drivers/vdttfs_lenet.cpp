// Task-1 driver: the LeNet-MNIST main() of the reference (T1V:242-320) on the
// MI355X engine.  Reads the reference's assets -- the weights blob and the
// flat MNIST test set ({i}.bin = 784 float32, label_onehot = N x 10 float32)
// -- runs encode -> conv/pool/FC layers -> argmin readout in batches, and
// prints the reference's summary.  The topology follows the blob: every
// 4-D (HWIO) layer is a valid convolution followed by a 2x2 min pool
// (T1V:295-301), every 2-D layer a fully connected layer.
//
//   vdttfs_lenet [--weights exported_models/snn_weights.bin]
//                [--data dataset_downloaded/mnist_test10k/] [--n 10000] [--batch N]
//                [--T 80] [--delta 16] [--encode log|linear] [--tc-in 17.452274] [--td-in 0]
#include "driver_util.h"

int main(int argc, char** argv) {
    const Args a(argc, argv);
    const int N = a.i("n", 10000);
    const int B = a.i("batch", N);
    const std::string weights = a.s("weights", "exported_models/snn_weights.bin");
    std::string dir = a.s("data", "dataset_downloaded/mnist_test10k/");
    if (!dir.empty() && dir.back() != '/') dir += '/';
    if (N <= 0 || B <= 0) {
        std::cerr << "--n and --batch must be positive" << std::endl;
        return 2;
    }
    const vdttfs_consts c = {a.i("T", 80), a.f("tfs", 0.0f), a.i("delta", 16), 1.0f,
                             /*alpha_by_time=*/0, /*conv_same_pad=*/0};
    const bool linear = a.s("encode", "log") == "linear";
    const float tc_in = a.f("tc-in", 17.452274f), td_in = a.f("td-in", 0.0f);

    std::cout << ">>> Loading LeNet-MNIST weights..." << std::endl;
    vdttfs_blob* blob = nullptr;
    VD_CHECK(vdttfs_blob_read(weights.c_str(), &blob));
    std::vector<vdttfs_layer_desc> L;
    int H = 28, W = 28, C = 1;
    for (int i = 0; i < blob->num_layers; ++i) {
        const vdttfs_blob_layer& b = blob->layers[i];
        vdttfs_layer_desc d{};
        d.kernel = b.kernel;
        d.bias = b.bias;
        d.tc_fire = b.tc_fire;
        d.td = b.td;
        if (b.ndim == 4) {
            if (b.c_in != C || b.k_h > H || b.k_w > W) {
                std::cerr << "layer " << i << ": conv does not fit its input" << std::endl;
                return 1;
            }
            d.kind = VDTTFS_LAYER_CONV;
            d.H_in = H, d.W_in = W, d.C_in = C;
            d.H_out = H - b.k_h + 1, d.W_out = W - b.k_w + 1, d.C_out = b.c_out;
            d.K_h = b.k_h, d.K_w = b.k_w;
            L.push_back(d);
            vdttfs_layer_desc p{};
            p.kind = VDTTFS_LAYER_POOL;
            p.H_in = d.H_out, p.W_in = d.W_out, p.C_in = d.C_out;
            p.H_out = d.H_out / 2, p.W_out = d.W_out / 2, p.C_out = d.C_out;
            L.push_back(p);
            H = p.H_out, W = p.W_out, C = p.C_out;
        } else {
            if (b.c_in != H * W * C) {
                std::cerr << "layer " << i << ": FC takes " << b.c_in << " inputs, previous gives "
                          << H * W * C << std::endl;
                return 1;
            }
            d.kind = VDTTFS_LAYER_FC;
            d.H_in = H, d.W_in = W, d.C_in = C;
            d.H_out = 1, d.W_out = 1, d.C_out = b.c_out;
            d.K_h = d.K_w = 1;
            L.push_back(d);
            H = W = 1, C = b.c_out;
        }
    }
    const int n_cls = C;

    std::cout << ">>> Loading " << N << " MNIST test images..." << std::endl;
    std::vector<float> imgs((size_t)N * 784), labels((size_t)N * n_cls);
    for (int i = 0; i < N; ++i) read_exact(dir + std::to_string(i) + ".bin", &imgs[(size_t)i * 784], 784);
    read_exact(dir + "label_onehot", labels.data(), labels.size());

    vdttfs_ctx* ctx = nullptr;
    VD_CHECK(vdttfs_create(&c, 0, &ctx));
    vdttfs_net* net = nullptr;
    VD_CHECK(vdttfs_net_create(ctx, L.data(), (int)L.size(), B, 784,
                               linear ? VDTTFS_ENCODE_LINEAR : VDTTFS_ENCODE_LOG, tc_in, td_in,
                               VDTTFS_READOUT_ARGMIN, &net));
    vdttfs_blob_free(blob);
    std::vector<int32_t> pred((size_t)B);
    std::vector<float> batch((size_t)B * 784, 0.0f);
    int correct = 0;
    {
        DevBuf d_img(ctx, batch.size() * 4), d_pred(ctx, pred.size() * 4);
        std::cout << ">>> Running time-sorted early-exit inference (CHUNK=" << c.delta << ")..." << std::endl;
        const auto t0 = std::chrono::steady_clock::now();
        VD_CHECK(vdttfs_timer_begin(ctx));
        for (int s = 0; s < N; s += B) {
            const int nb = std::min(B, N - s);
            std::copy(imgs.begin() + (size_t)s * 784, imgs.begin() + (size_t)(s + nb) * 784, batch.begin());
            VD_CHECK(vdttfs_h2d(ctx, d_img.p, batch.data(), batch.size() * 4));
            VD_CHECK(vdttfs_net_forward(net, d_img.as<float>(), d_pred.as<int32_t>()));
            VD_CHECK(vdttfs_d2h(ctx, pred.data(), d_pred.p, pred.size() * 4));
            for (int k = 0; k < nb; ++k)
                if (pred[k] == onehot_class(&labels[(size_t)(s + k) * n_cls], n_cls)) ++correct;
        }
        double ms = 0;
        VD_CHECK(vdttfs_timer_end(ctx, &ms));
        const double wall = seconds_since(t0);
        std::cout << "\n=======================================" << std::endl;
        std::cout << "TIME-SORTED EARLY-EXIT (LeNet-MNIST) COMPLETED" << std::endl;
        std::cout << "Images Processed:     " << N << std::endl;
        std::cout << "Final Accuracy:       " << (float)correct / N * 100.0f << "%" << std::endl;
        std::cout << "Total Inference Time: " << ms / 1000.0 << " seconds" << std::endl;
        std::cout << "Throughput:           " << N / (ms / 1000.0) << " images/sec" << std::endl;
        std::cout << "Host wall time:       " << wall << " seconds" << std::endl;
        std::cout << "=======================================" << std::endl;
    }
    vdttfs_net_destroy(net);
    vdttfs_destroy(ctx);
    return 0;
}
