// Task-3 driver: the DVSGesture main() of the reference (T3V:234-300) on the
// MI355X CuLIF engine.  Reads the reference's assets -- one flat float32
// weights file (conv1 OIHW, conv2, conv3, fc1_rec [128][128], fc1
// [128][128*(H/4)*(W/4)], fc2 [classes][128], in that order: the offsets of
// T3V:241-243), the dense event tensor train_data.bin (N x 2 x H x W x T
// float32) and train_labels.bin (N x classes int32 one-hot) -- runs the
// 7-layer network (conv 2->64 on raw events, conv 64->128, pool, conv
// 128->128, pool, recurrent fc1, fc2) and the argmin readout, and prints the
// reference's summary.  Defaults are T3V's constants (T3V:17-27).
//
//   vdttfs_dvs [--weights cuda_assets/dvsgesture_weights.bin]
//              [--data cuda_assets/train_data.bin] [--labels cuda_assets/train_labels.bin]
//              [--n 1078] [--batch N] [--size 32] [--classes 10] [--T 160] [--delta 32]
//              [--decay-conv exp(-1/5)] [--th-conv 5] [--decay-fc exp(-1/60)] [--th-fc 10]
#include <cmath>
#include <iomanip>

#include "driver_util.h"

int main(int argc, char** argv) {
    const Args a(argc, argv);
    const int N = a.i("n", 1078);
    const int B = a.i("batch", N);
    const int S = a.i("size", 32);
    const int n_cls = a.i("classes", 10);
    const int T = a.i("T", 160);
    const std::string wpath = a.s("weights", "cuda_assets/dvsgesture_weights.bin");
    const std::string dpath = a.s("data", "cuda_assets/train_data.bin");
    const std::string lpath = a.s("labels", "cuda_assets/train_labels.bin");
    if (N <= 0 || B <= 0 || S < 4 || S % 4 != 0 || n_cls <= 0) {
        std::cerr << "bad --n / --batch / --size / --classes" << std::endl;
        return 2;
    }
    // T3V:24-27: decays computed in float as the reference's constants are
    const float decay_conv = a.f("decay-conv", (float)std::exp((double)(-1.0f / 5.0f)));
    const float decay_fc = a.f("decay-fc", (float)std::exp((double)(-1.0f / 60.0f)));
    const float th_conv = a.f("th-conv", 5.0f), th_fc = a.f("th-fc", 10.0f);
    const vdttfs_consts c = {T, 0.0f, a.i("delta", 32), 1.0f, 0, 1};

    std::cout << ">>> VD-TTFS time-sorted (bucketized) chunked early-exit, DVSGesture..." << std::endl;
    const int F = 128 * (S / 4) * (S / 4);
    const size_t n1 = 64 * 2 * 9, n2 = 128 * 64 * 9, n3 = 128 * 128 * 9, nr = 128 * 128,
                 nf1 = (size_t)128 * F, nf2 = (size_t)n_cls * 128;
    std::vector<float> w(n1 + n2 + n3 + nr + nf1 + nf2);
    read_exact(wpath, w.data(), w.size());
    const float* w_conv1 = w.data();
    const float* w_conv2 = w_conv1 + n1;
    const float* w_conv3 = w_conv2 + n2;
    const float* w_rec = w_conv3 + n3;
    const float* w_fc1 = w_rec + nr;
    const float* w_fc2 = w_fc1 + nf1;

    const size_t per = (size_t)2 * S * S * T;
    std::vector<float> data((size_t)N * per);
    read_exact(dpath, data.data(), data.size());
    std::vector<int32_t> labels((size_t)N * n_cls);
    read_exact(lpath, labels.data(), labels.size());

    const vdttfs_culif_layer L[7] = {
        {VDTTFS_CULIF_RAW_CONV, 2, S, S, 64, w_conv1, nullptr, decay_conv, th_conv},
        {VDTTFS_CULIF_CONV, 64, S, S, 128, w_conv2, nullptr, decay_conv, th_conv},
        {VDTTFS_CULIF_POOL, 128, S, S, 128, nullptr, nullptr, decay_conv, th_conv},
        {VDTTFS_CULIF_CONV, 128, S / 2, S / 2, 128, w_conv3, nullptr, decay_conv, th_conv},
        {VDTTFS_CULIF_POOL, 128, S / 2, S / 2, 128, nullptr, nullptr, decay_conv, th_conv},
        {VDTTFS_CULIF_FC_REC, F, 1, 1, 128, w_fc1, w_rec, decay_fc, th_fc},
        {VDTTFS_CULIF_FC, 128, 1, 1, n_cls, w_fc2, nullptr, decay_fc, th_fc},
    };
    vdttfs_ctx* ctx = nullptr;
    VD_CHECK(vdttfs_create(&c, 0, &ctx));
    vdttfs_culif_net* net = nullptr;
    VD_CHECK(vdttfs_culif_net_create(ctx, L, 7, B, &net));
    std::vector<int32_t> pred((size_t)B);
    std::vector<float> batch((size_t)B * per, 0.0f);
    int correct = 0;
    double ms_total = 0;
    {
        DevBuf d_data(ctx, batch.size() * 4), d_pred(ctx, pred.size() * 4);
        for (int s = 0; s < N; s += B) {
            const int nb = std::min(B, N - s);
            std::copy(data.begin() + (size_t)s * per, data.begin() + (size_t)(s + nb) * per, batch.begin());
            VD_CHECK(vdttfs_h2d(ctx, d_data.p, batch.data(), batch.size() * 4));
            // timed as T3V:270-289: the layers with the events already on the device
            VD_CHECK(vdttfs_timer_begin(ctx));
            VD_CHECK(vdttfs_culif_net_forward(net, d_data.as<float>(), d_pred.as<int32_t>()));
            double ms = 0;
            VD_CHECK(vdttfs_timer_end(ctx, &ms));
            ms_total += ms;
            VD_CHECK(vdttfs_d2h(ctx, pred.data(), d_pred.p, pred.size() * 4));
            for (int k = 0; k < nb; ++k) {
                // T3V:283-285: truth = first maximal label entry
                const int32_t* lr = &labels[(size_t)(s + k) * n_cls];
                int truth = 0, mg = lr[0];
                for (int q = 1; q < n_cls; ++q)
                    if (lr[q] > mg) {
                        mg = lr[q];
                        truth = q;
                    }
                if (pred[k] == truth) ++correct;
            }
        }
    }
    std::cout << "=================================================" << std::endl;
    std::cout << "Inference time:  " << ms_total << " ms" << std::endl;
    std::cout << "Throughput:      " << (N * 1000.0) / ms_total << " samples/sec" << std::endl;
    std::cout << "Accuracy:        " << std::fixed << std::setprecision(2) << (float)correct / N * 100.0f << " %" << std::endl;
    std::cout << "=================================================" << std::endl;
    vdttfs_culif_net_destroy(net);
    vdttfs_destroy(ctx);
    return 0;
}
