// core_module.cpp -- the msplat._core extension: TrainingConfig,
// TrainingStats, Dataset, GaussianTrainer, sync, cleanup, with the
// signatures, defaults and errors of the reference's nanobind module
// (python/bindings.cpp:24-418, stubs python/msplat/_core.pyi), built with
// pybind11 over the C++ trainer API (include/msplat_api.hpp).
#include <pybind11/functional.h>
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "input_data.hpp"
#include "model.hpp"
#include "msplat_api.hpp"

namespace py = pybind11;
using namespace pybind11::literals;

namespace {

struct TrainingConfig {
    int iterations = 30000;
    int sh_degree = 3;
    int sh_degree_interval = 1000;
    float ssim_weight = 0.2f;
    int num_downscales = 2;
    int resolution_schedule = 3000;
    int refine_every = 100;
    int warmup_length = 500;
    int reset_alpha_every = 30;
    float densify_grad_thresh = 0.0002f;
    float densify_size_thresh = 0.01f;
    int stop_screen_size_at = 4000;
    float split_screen_size = 0.05f;
    bool keep_crs = false;
    float downscale_factor = 1.0f;
    std::string output = "splat.ply";
    int save_every = -1;
    std::vector<float> bg_color = {0.6130f, 0.0101f, 0.3984f};

    msplat::Config to_config() const {
        if (bg_color.size() != 3) throw py::value_error("bg_color must have exactly 3 elements [R, G, B]");
        msplat::Config c;
        c.iterations = iterations;
        c.shDegree = sh_degree;
        c.shDegreeInterval = sh_degree_interval;
        c.ssimWeight = ssim_weight;
        c.numDownscales = num_downscales;
        c.resolutionSchedule = resolution_schedule;
        c.refineEvery = refine_every;
        c.warmupLength = warmup_length;
        c.resetAlphaEvery = reset_alpha_every;
        c.densifyGradThresh = densify_grad_thresh;
        c.densifySizeThresh = densify_size_thresh;
        c.stopScreenSizeAt = stop_screen_size_at;
        c.splitScreenSize = split_screen_size;
        c.keepCrs = keep_crs;
        c.downscaleFactor = downscale_factor;
        for (int i = 0; i < 3; ++i) c.bgColor[i] = bg_color[i];
        return c;
    }
};

struct TrainingStats {
    int iteration = 0;
    int splat_count = 0;
    float ms_per_step = 0.f;
    float loss = 0.f;
};

py::array_t<float> to_numpy(msplat::PixelBuffer &&b) {
    if (!b.data) throw std::runtime_error("render produced no image");
    py::array_t<float> a({(py::ssize_t)b.height, (py::ssize_t)b.width, (py::ssize_t)3});
    std::memcpy(a.mutable_data(), b.data, (size_t)b.width * b.height * 3 * sizeof(float));
    return a;
}

struct Trainer {
    msplat::Trainer t;
    TrainingConfig config;
    int num_train, num_test;
    Trainer(msplat::Dataset &ds, const TrainingConfig &cfg, const std::string &primitive)
        : t(ds, cfg.to_config(), parse_primitive(primitive)),
          config(cfg),
          num_train(ds.numTrain()),
          num_test(ds.numTest()) {}
    static msplat::Primitive parse_primitive(const std::string &p) {
        if (p == "2dgs") return msplat::Primitive::Surfel2D;
        if (p == "3dgs") return msplat::Primitive::Gaussian3D;
        throw std::invalid_argument("primitive must be '2dgs' or '3dgs'");
    }
};

TrainingStats to_stats(const msplat::Stats &s) {
    TrainingStats o;
    o.iteration = s.iteration;
    o.splat_count = s.splatCount;
    o.ms_per_step = s.msPerStep;
    o.loss = s.loss;
    return o;
}

}  // namespace

PYBIND11_MODULE(_core, m) {
    m.doc() = "msplat: 2D Gaussian Splatting training on AMD Instinct MI355X (gfx950 HIP kernels)";

    py::class_<TrainingConfig>(m, "TrainingConfig")
        .def(py::init([](int iterations, int sh_degree, int sh_degree_interval, float ssim_weight,
                         int num_downscales, int resolution_schedule, int refine_every, int warmup_length,
                         int reset_alpha_every, float densify_grad_thresh, float densify_size_thresh,
                         int stop_screen_size_at, float split_screen_size, bool keep_crs, float downscale_factor,
                         const std::string &output, int save_every, std::vector<float> bg_color) {
                 if (bg_color.size() != 3) throw py::value_error("bg_color must have exactly 3 elements [R, G, B]");
                 TrainingConfig c;
                 c.iterations = iterations;
                 c.sh_degree = sh_degree;
                 c.sh_degree_interval = sh_degree_interval;
                 c.ssim_weight = ssim_weight;
                 c.num_downscales = num_downscales;
                 c.resolution_schedule = resolution_schedule;
                 c.refine_every = refine_every;
                 c.warmup_length = warmup_length;
                 c.reset_alpha_every = reset_alpha_every;
                 c.densify_grad_thresh = densify_grad_thresh;
                 c.densify_size_thresh = densify_size_thresh;
                 c.stop_screen_size_at = stop_screen_size_at;
                 c.split_screen_size = split_screen_size;
                 c.keep_crs = keep_crs;
                 c.downscale_factor = downscale_factor;
                 c.output = output;
                 c.save_every = save_every;
                 c.bg_color = std::move(bg_color);
                 return c;
             }),
             "iterations"_a = 30000, "sh_degree"_a = 3, "sh_degree_interval"_a = 1000, "ssim_weight"_a = 0.2f,
             "num_downscales"_a = 2, "resolution_schedule"_a = 3000, "refine_every"_a = 100, "warmup_length"_a = 500,
             "reset_alpha_every"_a = 30, "densify_grad_thresh"_a = 0.0002f, "densify_size_thresh"_a = 0.01f,
             "stop_screen_size_at"_a = 4000, "split_screen_size"_a = 0.05f, "keep_crs"_a = false,
             "downscale_factor"_a = 1.0f, "output"_a = "splat.ply", "save_every"_a = -1,
             "bg_color"_a = std::vector<float>{0.6130f, 0.0101f, 0.3984f})
        .def_readwrite("iterations", &TrainingConfig::iterations)
        .def_readwrite("sh_degree", &TrainingConfig::sh_degree)
        .def_readwrite("sh_degree_interval", &TrainingConfig::sh_degree_interval)
        .def_readwrite("ssim_weight", &TrainingConfig::ssim_weight)
        .def_readwrite("num_downscales", &TrainingConfig::num_downscales)
        .def_readwrite("resolution_schedule", &TrainingConfig::resolution_schedule)
        .def_readwrite("refine_every", &TrainingConfig::refine_every)
        .def_readwrite("warmup_length", &TrainingConfig::warmup_length)
        .def_readwrite("reset_alpha_every", &TrainingConfig::reset_alpha_every)
        .def_readwrite("densify_grad_thresh", &TrainingConfig::densify_grad_thresh)
        .def_readwrite("densify_size_thresh", &TrainingConfig::densify_size_thresh)
        .def_readwrite("stop_screen_size_at", &TrainingConfig::stop_screen_size_at)
        .def_readwrite("split_screen_size", &TrainingConfig::split_screen_size)
        .def_readwrite("keep_crs", &TrainingConfig::keep_crs)
        .def_readwrite("downscale_factor", &TrainingConfig::downscale_factor)
        .def_readwrite("output", &TrainingConfig::output)
        .def_readwrite("save_every", &TrainingConfig::save_every)
        .def_property(
            "bg_color", [](const TrainingConfig &c) { return c.bg_color; },
            [](TrainingConfig &c, std::vector<float> v) {
                if (v.size() != 3) throw py::value_error("bg_color must have exactly 3 elements [R, G, B]");
                c.bg_color = std::move(v);
            },
            "Background color as [R, G, B] floats in [0, 1]. Default magenta [0.613, 0.010, 0.398].");

    py::class_<TrainingStats>(m, "TrainingStats", "Per-step training statistics returned by GaussianTrainer.step().")
        .def_readonly("iteration", &TrainingStats::iteration, "Current training iteration.")
        .def_readonly("splat_count", &TrainingStats::splat_count, "Number of active Gaussians.")
        .def_readonly("ms_per_step", &TrainingStats::ms_per_step, "Wall-clock time for this step in milliseconds.")
        .def_readonly("loss", &TrainingStats::loss, "Training loss of this step (L1 + D-SSIM).")
        .def("__repr__", [](const TrainingStats &s) {
            return "TrainingStats(iteration=" + std::to_string(s.iteration) +
                   ", splats=" + std::to_string(s.splat_count) + ", ms=" + std::to_string(s.ms_per_step) + ")";
        });

    py::class_<msplat::Dataset>(m, "Dataset",
                                "A loaded dataset of camera images. Auto-detects COLMAP, Nerfstudio, and Polycam "
                                "formats.")
        .def(py::init<const std::string &, float, bool, int>(), "path"_a, "downscale_factor"_a = 1.0f,
             "eval_mode"_a = false, "test_every"_a = 8)
        .def_static(
            "from_arrays",
            [](const std::vector<py::array_t<float, py::array::c_style | py::array::forcecast>> &images,
               py::array_t<float, py::array::c_style | py::array::forcecast> cam_to_world,
               py::array_t<float, py::array::c_style | py::array::forcecast> intrinsics, py::object points_xyz,
               py::object points_rgb, bool eval_mode, int test_every) {
                const size_t n = images.size();
                if (n == 0) throw py::value_error("no images");
                if (cam_to_world.ndim() != 3 || (size_t)cam_to_world.shape(0) != n || cam_to_world.shape(1) != 4 ||
                    cam_to_world.shape(2) != 4)
                    throw py::value_error("cam_to_world must have shape (N, 4, 4)");
                if (intrinsics.ndim() != 2 || (size_t)intrinsics.shape(0) != n || intrinsics.shape(1) != 4)
                    throw py::value_error("intrinsics must have shape (N, 4): fx, fy, cx, cy");
                std::vector<msplat::CameraImage> cams(n);
                for (size_t i = 0; i < n; ++i) {
                    const auto &im = images[i];
                    if (im.ndim() != 3 || im.shape(2) != 3) throw py::value_error("images must be (H, W, 3) float32");
                    cams[i].height = (int)im.shape(0);
                    cams[i].width = (int)im.shape(1);
                    const float *k = intrinsics.data() + 4 * i;
                    cams[i].fx = k[0];
                    cams[i].fy = k[1];
                    cams[i].cx = k[2];
                    cams[i].cy = k[3];
                    std::memcpy(cams[i].camToWorld, cam_to_world.data() + 16 * i, 16 * sizeof(float));
                    cams[i].rgb = im.data();
                }
                std::vector<float> xyz;
                std::vector<uint8_t> rgb;
                int64_t np_ = 0;
                if (!points_xyz.is_none()) {
                    auto a = py::array_t<float, py::array::c_style | py::array::forcecast>::ensure(points_xyz);
                    auto c = py::array_t<uint8_t, py::array::c_style | py::array::forcecast>::ensure(points_rgb);
                    if (!a || a.ndim() != 2 || a.shape(1) != 3) throw py::value_error("points_xyz must be (P, 3)");
                    if (!c || c.ndim() != 2 || c.shape(0) != a.shape(0) || c.shape(1) != 3)
                        throw py::value_error("points_rgb must be (P, 3) uint8");
                    np_ = a.shape(0);
                    xyz.assign(a.data(), a.data() + 3 * np_);
                    rgb.assign(c.data(), c.data() + 3 * np_);
                }
                return new msplat::Dataset(cams, xyz.data(), rgb.data(), np_, eval_mode, test_every);
            },
            "images"_a, "cam_to_world"_a, "intrinsics"_a, "points_xyz"_a = py::none(), "points_rgb"_a = py::none(),
            "eval_mode"_a = false, "test_every"_a = 8,
            "Dataset from in-memory (H, W, 3) float32 images, (N, 4, 4) camera-to-world poses (OpenGL axes) and "
            "(N, 4) intrinsics fx, fy, cx, cy; optional initial point cloud (P, 3) float32 + (P, 3) uint8.")
        .def_property_readonly("num_train", &msplat::Dataset::numTrain, "Number of training cameras.")
        .def_property_readonly("num_test", &msplat::Dataset::numTest,
                               "Number of test cameras (0 unless eval_mode=True).")
        .def(
            "camera_pose",
            [](const msplat::Dataset &d, int index) {
                if (index < 0 || index >= d.numTrain()) throw std::runtime_error("Camera index out of range");
                py::array_t<float> a({4, 4});
                d.cameraPose(index, a.mutable_data());
                return a;
            },
            "index"_a, "Get camera-to-world pose (4x4 row-major, OpenGL convention) as numpy array.");

    py::class_<Trainer>(m, "GaussianTrainer", "Gaussian Splatting trainer (2DGS surfels, or 3D Gaussians with primitive='3dgs'). All computation runs on the GPU.")
        .def(py::init<msplat::Dataset &, const TrainingConfig &, const std::string &>(), "dataset"_a, "config"_a,
             "primitive"_a = "2dgs", py::keep_alive<1, 2>(),
             "primitive: '2dgs' (surfels, the default) or '3dgs' (3D Gaussians; no mesh or point-cloud export).")
        .def_property_readonly(
            "primitive",
            [](const Trainer &t) { return t.t.primitive() == msplat::Primitive::Gaussian3D ? "3dgs" : "2dgs"; })
        .def(
            "step", [](Trainer &t) { return to_stats(t.t.step()); },
            "Run a single training iteration. Returns TrainingStats.")
        .def(
            "train",
            [](Trainer &t, py::object callback, int callback_every) {
                while (t.t.iteration() < t.config.iterations) {
                    const TrainingStats s = to_stats(t.t.step());
                    if (callback_every > 0 && s.iteration % callback_every == 0 && !callback.is_none()) callback(s);
                }
            },
            "callback"_a, "callback_every"_a = 100,
            "Run training to completion, calling callback(stats) every callback_every steps.")
        .def(
            "evaluate",
            [](Trainer &t) {
                if (t.num_test == 0) throw std::runtime_error("No test cameras. Load dataset with eval_mode=True.");
                const msplat::EvalMetrics e = t.t.evaluate();
                py::dict d;
                d["psnr"] = e.psnr;
                d["ssim"] = e.ssim;
                d["l1"] = e.l1;
                d["num_test"] = e.numTest;
                d["num_gaussians"] = e.numGaussians;
                return d;
            },
            "Evaluate on held-out test cameras. Returns dict with psnr, ssim, l1 keys.\n"
            "Requires the dataset to have been loaded with eval_mode=True.")
        .def(
            "render",
            [](Trainer &t, int cam_idx, bool use_test) {
                const int n = use_test ? t.num_test : t.num_train;
                if (cam_idx < 0 || cam_idx >= n) throw std::runtime_error("Camera index out of range");
                return to_numpy(t.t.render(cam_idx, use_test));
            },
            "cam_idx"_a, "use_test"_a = false,
            "Render a camera view. Returns a numpy array of shape (H, W, 3), float32, RGB [0,1].")
        .def(
            "render_from_pose",
            [](Trainer &t, py::array_t<float, py::array::c_style | py::array::forcecast> cam_to_world,
               int ref_cam_idx) {
                if (cam_to_world.size() != 16)
                    throw std::runtime_error("cam_to_world must have 16 elements (4x4 matrix)");
                if (ref_cam_idx < 0 || ref_cam_idx >= t.num_train) throw std::runtime_error("ref_cam_idx out of range");
                return to_numpy(t.t.renderFromPose(cam_to_world.data(), ref_cam_idx));
            },
            "cam_to_world"_a, "ref_cam_idx"_a = 0,
            "Render from an arbitrary camera-to-world pose (4x4 row-major, OpenGL convention).\n"
            "Uses intrinsics from ref_cam_idx. Returns numpy (H, W, 3) float32.")
        .def(
            "export_ply", [](Trainer &t, const std::string &p) { t.t.exportPly(p); }, "path"_a,
            "Export the current Gaussians as a PLY file.")
        .def(
            "export_splat", [](Trainer &t, const std::string &p) { t.t.exportSplat(p); }, "path"_a,
            "Export the current Gaussians as a .splat file.")
        .def(
            "extract_mesh",
            [](Trainer &t, const std::string &p, float voxel_size, float bound_radius, float alpha_thresh,
               float trunc_multiplier) {
                return t.t.extractMesh(p, voxel_size, bound_radius, alpha_thresh, trunc_multiplier);
            },
            "path"_a, "voxel_size"_a = 0.004f, "bound_radius"_a = 0.3f, "alpha_thresh"_a = 0.5f,
            "trunc_multiplier"_a = 4.0f,
            "TSDF fusion of the training views + marching cubes; writes a triangle PLY, returns the triangle count.")
        .def(
            "export_point_cloud",
            [](Trainer &t, const std::string &p, float alpha_thresh) { return t.t.exportPointCloud(p, alpha_thresh); },
            "path"_a, "alpha_thresh"_a = 0.5f,
            "Unproject every training view's depth into a coloured PLY point cloud; returns the point count.")
        .def(
            "save_checkpoint", [](Trainer &t, const std::string &p) { t.t.saveCheckpoint(p); }, "path"_a,
            "Save a training checkpoint.")
        .def(
            "load_checkpoint", [](Trainer &t, const std::string &p) { t.t.loadCheckpoint(p); }, "path"_a,
            "Load a training checkpoint and resume from the saved iteration.")
        .def(
            "load_ply", [](Trainer &t, const std::string &p) { return t.t.loadPly(p); }, "path"_a,
            "Replace the scene with a Gaussian PLY and resume at the step it records.")
        .def(
            "set_max_splats", [](Trainer &t, int n) { t.t.setMaxSplats(n); }, "max_splats"_a,
            "Densification cap (250000 by default).")
        .def(
            "set_cull_alpha", [](Trainer &t, float a) { t.t.setCullAlphaThresh(a); }, "thresh"_a,
            "Cull threshold on sigmoid(opacity) used by densification (0.1 by default).")
        .def_property_readonly(
            "splat_count", [](const Trainer &t) { return t.t.splatCount(); }, "Current number of active Gaussians.")
        .def_property_readonly(
            "iteration", [](const Trainer &t) { return t.t.iteration(); }, "Current training iteration.");

    m.def(
        "_read_image",
        [](const std::string &path) {
            const Image im = imreadRGB(path);
            py::array_t<float> a({(py::ssize_t)im.height, (py::ssize_t)im.width, (py::ssize_t)3});
            std::memcpy(a.mutable_data(), im.ptr(), im.data.size() * sizeof(float));
            return a;
        },
        "path"_a, "Decode an image file the way datasets do (PNG / PPM / PGM / JPEG) to (H, W, 3) float32 in [0, 1].");
    m.def(
        "_metrics",
        [](py::array_t<float, py::array::c_style | py::array::forcecast> rendered,
           py::array_t<float, py::array::c_style | py::array::forcecast> gt) {
            if (rendered.ndim() != 3 || gt.ndim() != 3) throw std::invalid_argument("images are (H, W, C)");
            auto host = [](const py::array_t<float, py::array::c_style | py::array::forcecast> &a) {
                MTensor t({(int64_t)a.shape(0), (int64_t)a.shape(1), (int64_t)a.shape(2)}, DType::Float32);
                std::memcpy(t.data<float>(), a.data(), (size_t)a.size() * sizeof(float));
                return t;
            };
            const MTensor r = host(rendered), g = host(gt);
            py::dict d;
            d["psnr"] = psnr(r, g);
            d["ssim"] = ssim_eval(r, g);
            d["l1"] = l1_loss(r, g);
            return d;
        },
        "rendered"_a, "gt"_a,
        "The evaluation metrics Trainer.evaluate reports (PSNR, SSIM with an 11-tap sigma-1.5 window and "
        "clamp-to-edge padding, L1) of two (H, W, C) float32 images on the host.");
    m.def("sync", &msplat::sync, "Synchronize GPU (wait for all commands to complete)");
    m.def("cleanup", &msplat::cleanup, "Release all cached GPU resources");
}
