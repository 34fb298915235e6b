// loaders.cpp -- dataset loaders and point-cloud readers: Nerfstudio
// (transforms.json), COLMAP (sparse model, binary) and Polycam (per-frame
// camera JSONs or cameras.json), auto-detected by inputDataFromX
// (core/src/input_data.cpp:424-436, core/src/loaders/load_*.cpp of the
// reference).  Poses become 4x4 row-major camera-to-world matrices in
// OpenGL axes; the scene is then centred and scaled (autoScaleAndCenter).
// JSON is read by a small recursive-descent parser (numbers, strings,
// arrays, objects, true/false/null).
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <iostream>
#include <map>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "input_data.hpp"

namespace fs = std::filesystem;

namespace {

// ---------------------------------------------------------------- JSON --

struct Json {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0;
    std::string str;
    std::vector<Json> arr;
    std::map<std::string, Json> obj;

    bool has(const std::string &k) const { return kind == Obj && obj.count(k); }
    const Json &at(const std::string &k) const {
        auto it = obj.find(k);
        if (kind != Obj || it == obj.end()) throw std::runtime_error("JSON: missing key '" + k + "'");
        return it->second;
    }
    const Json &operator[](size_t i) const {
        if (kind != Arr || i >= arr.size()) throw std::runtime_error("JSON: index out of range");
        return arr[i];
    }
    double number() const {
        if (kind != Num) throw std::runtime_error("JSON: expected a number");
        return num;
    }
    double value(const std::string &k, double dflt) const { return has(k) ? at(k).number() : dflt; }
    std::string value(const std::string &k, const std::string &dflt) const {
        return has(k) && at(k).kind == Str ? at(k).str : dflt;
    }
};

class JsonParser {
public:
    explicit JsonParser(const std::string &s) : s_(s) {}
    Json parse() {
        Json v = value();
        ws();
        if (p_ != s_.size()) fail("trailing characters");
        return v;
    }

private:
    const std::string &s_;
    size_t p_ = 0;

    [[noreturn]] void fail(const char *what) {
        throw std::runtime_error(std::string("JSON parse error: ") + what + " at offset " + std::to_string(p_));
    }
    void ws() {
        while (p_ < s_.size() && std::isspace((unsigned char)s_[p_])) ++p_;
    }
    bool eat(char c) {
        ws();
        if (p_ < s_.size() && s_[p_] == c) {
            ++p_;
            return true;
        }
        return false;
    }
    Json value() {
        ws();
        if (p_ >= s_.size()) fail("unexpected end");
        const char c = s_[p_];
        Json v;
        if (c == '{') {
            ++p_;
            v.kind = Json::Obj;
            if (eat('}')) return v;
            do {
                ws();
                std::string k = string();
                if (!eat(':')) fail("expected ':'");
                v.obj[k] = value();
            } while (eat(','));
            if (!eat('}')) fail("expected '}'");
        } else if (c == '[') {
            ++p_;
            v.kind = Json::Arr;
            if (eat(']')) return v;
            do v.arr.push_back(value());
            while (eat(','));
            if (!eat(']')) fail("expected ']'");
        } else if (c == '"') {
            v.kind = Json::Str;
            v.str = string();
        } else if (!s_.compare(p_, 4, "true")) {
            p_ += 4;
            v.kind = Json::Bool;
            v.b = true;
        } else if (!s_.compare(p_, 5, "false")) {
            p_ += 5;
            v.kind = Json::Bool;
        } else if (!s_.compare(p_, 4, "null")) {
            p_ += 4;
        } else {
            char *end = nullptr;
            v.num = std::strtod(s_.c_str() + p_, &end);
            if (end == s_.c_str() + p_) fail("bad value");
            p_ = end - s_.c_str();
            v.kind = Json::Num;
        }
        return v;
    }
    std::string string() {
        if (p_ >= s_.size() || s_[p_] != '"') fail("expected string");
        ++p_;
        std::string out;
        while (p_ < s_.size() && s_[p_] != '"') {
            char c = s_[p_++];
            if (c == '\\') {
                if (p_ >= s_.size()) fail("bad escape");
                const char e = s_[p_++];
                switch (e) {
                    case 'n': out += '\n'; break;
                    case 't': out += '\t'; break;
                    case 'r': out += '\r'; break;
                    case 'b': out += '\b'; break;
                    case 'f': out += '\f'; break;
                    case 'u': {
                        if (p_ + 4 > s_.size()) fail("bad \\u escape");
                        const unsigned cp = (unsigned)std::stoul(s_.substr(p_, 4), nullptr, 16);
                        p_ += 4;
                        if (cp < 0x80) {
                            out += (char)cp;
                        } else if (cp < 0x800) {
                            out += (char)(0xC0 | (cp >> 6));
                            out += (char)(0x80 | (cp & 0x3F));
                        } else {
                            out += (char)(0xE0 | (cp >> 12));
                            out += (char)(0x80 | ((cp >> 6) & 0x3F));
                            out += (char)(0x80 | (cp & 0x3F));
                        }
                        break;
                    }
                    default: out += e;
                }
            } else {
                out += c;
            }
        }
        if (p_ >= s_.size()) fail("unterminated string");
        ++p_;
        return out;
    }
};

Json read_json(const fs::path &p) {
    std::ifstream f(p);
    if (!f) throw std::runtime_error("cannot open " + p.string());
    std::stringstream ss;
    ss << f.rdbuf();
    const std::string s = ss.str();
    return JsonParser(s).parse();
}

std::string resolve_image(const std::string &path) {
    if (fs::exists(path)) return path;
    for (const char *ext : {".png", ".jpg", ".jpeg", ".JPG", ".ppm"})
        if (fs::exists(path + ext)) return path + ext;
    return path;
}

void read_matrix4(const Json &m, float out[16]) {
    for (int r = 0; r < 4; ++r)
        for (int c = 0; c < 4; ++c) out[4 * r + c] = (float)m[r][c].number();
}

// ------------------------------------------------------------ Nerfstudio --

InputData load_nerfstudio(const std::string &root) {
    const Json j = read_json(fs::path(root) / "transforms.json");
    const int gW = (int)j.value("w", 0.0), gH = (int)j.value("h", 0.0);
    const float gFx = (float)j.value("fl_x", 0.0), gFy = (float)j.value("fl_y", 0.0);
    const bool haveCAX = j.has("camera_angle_x"), haveCAY = j.has("camera_angle_y");
    const float cax = (float)j.value("camera_angle_x", 0.0), cay = (float)j.value("camera_angle_y", 0.0);
    const bool haveCx = j.has("cx"), haveCy = j.has("cy");
    const float gCx = (float)j.value("cx", 0.0), gCy = (float)j.value("cy", 0.0);
    const float gK1 = (float)j.value("k1", 0.0), gK2 = (float)j.value("k2", 0.0), gK3 = (float)j.value("k3", 0.0);
    const float gP1 = (float)j.value("p1", 0.0), gP2 = (float)j.value("p2", 0.0);
    InputData data;
    for (const Json &fr : j.at("frames").arr) {
        Camera cam;
        cam.width = (int)fr.value("w", (double)gW);
        cam.height = (int)fr.value("h", (double)gH);
        cam.fx = (float)fr.value("fl_x", gFx);
        cam.fy = (float)fr.value("fl_y", gFy);
        cam.cx = fr.has("cx") ? (float)fr.at("cx").number() : (haveCx ? gCx : -1.0f);
        cam.cy = fr.has("cy") ? (float)fr.at("cy").number() : (haveCy ? gCy : -1.0f);
        cam.k1 = (float)fr.value("k1", gK1);
        cam.k2 = (float)fr.value("k2", gK2);
        cam.k3 = (float)fr.value("k3", gK3);
        cam.p1 = (float)fr.value("p1", gP1);
        cam.p2 = (float)fr.value("p2", gP2);
        const std::string fp = fr.at("file_path").str;
        cam.filePath = (!fp.empty() && (fp[0] == '/' || fp[0] == '.')) ? resolve_image(fp)
                                                                       : resolve_image((fs::path(root) / fp).string());
        read_matrix4(fr.at("transform_matrix"), cam.camToWorld);
        data.cameras.push_back(std::move(cam));
    }
    std::sort(data.cameras.begin(), data.cameras.end(),
              [](const Camera &a, const Camera &b) { return a.filePath < b.filePath; });
    // missing intrinsics: derive from the first image and camera_angle_x/y
    bool derive = false;
    for (auto &c : data.cameras)
        if (c.width <= 0 || c.height <= 0 || c.fx <= 0 || c.fy <= 0) derive = true;
    if (derive && !data.cameras.empty()) {
        const Image probe = imreadRGB(data.cameras.front().filePath);
        for (auto &c : data.cameras) {
            if (c.width <= 0) c.width = probe.width;
            if (c.height <= 0) c.height = probe.height;
            if (c.fx <= 0) {
                const float ang = haveCAX ? cax : (haveCAY ? cay : 0.0f);
                if (ang > 0) c.fx = (float)c.width * 0.5f / std::tan(0.5f * ang);
            }
            if (c.fy <= 0) c.fy = haveCAY ? (float)c.height * 0.5f / std::tan(0.5f * cay) : c.fx;
        }
    }
    for (auto &c : data.cameras) {
        if (c.cx < 0) c.cx = (float)c.width * 0.5f;
        if (c.cy < 0) c.cy = (float)c.height * 0.5f;
    }
    if (j.has("ply_file_path")) {
        std::string p = j.at("ply_file_path").str;
        if (!p.empty() && p[0] != '/') p = (fs::path(root) / p).string();
        if (fs::exists(p)) data.points = readPly(p);
    }
    if (data.points.count == 0)
        for (const char *p : {"sparse/0/points3D.ply", "points3D.ply", "points3d.ply"}) {
            const fs::path q = fs::path(root) / p;
            if (fs::exists(q)) {
                data.points = readPly(q.string());
                break;
            }
        }
    const char *face = std::getenv("MSPLAT_FACE_DISTANCE");
    if (face && std::atof(face) > 0.0) {
        const char *sf = std::getenv("MSPLAT_SCALE_FACTOR");
        const float scale = sf ? (float)std::atof(sf) : 10.0f;
        std::cerr << "msplat: face-centred transform (face distance " << std::atof(face) << ", scale " << scale
                  << ")\n";
        faceCenteredTransform(data, (float)std::atof(face), scale);
    } else {
        autoScaleAndCenter(data);
    }
    return data;
}

// ---------------------------------------------------------------- COLMAP --

struct ColmapCam {
    int model = 0, width = 0, height = 0;
    float fx = 0, fy = 0, cx = 0, cy = 0, k1 = 0, k2 = 0, p1 = 0, p2 = 0;
};

template <typename T>
T rd(std::ifstream &f) {
    T v{};
    f.read((char *)&v, sizeof(T));
    if (!f) throw std::runtime_error("COLMAP: truncated binary file");
    return v;
}

std::unordered_map<uint32_t, ColmapCam> read_cameras_bin(const std::string &path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open " + path);
    const uint64_t n = rd<uint64_t>(f);
    std::unordered_map<uint32_t, ColmapCam> cams;
    for (uint64_t i = 0; i < n; ++i) {
        ColmapCam c;
        const uint32_t id = rd<uint32_t>(f);
        c.model = (int)rd<int32_t>(f);
        c.width = (int)rd<uint64_t>(f);
        c.height = (int)rd<uint64_t>(f);
        auto d = [&] { return (float)rd<double>(f); };
        switch (c.model) {
            case 0: c.fx = c.fy = d(); c.cx = d(); c.cy = d(); break;                               // SIMPLE_PINHOLE
            case 1: c.fx = d(); c.fy = d(); c.cx = d(); c.cy = d(); break;                          // PINHOLE
            case 2: c.fx = c.fy = d(); c.cx = d(); c.cy = d(); c.k1 = d(); break;                   // SIMPLE_RADIAL
            case 3: c.fx = c.fy = d(); c.cx = d(); c.cy = d(); c.k1 = d(); c.k2 = d(); break;       // RADIAL
            case 4:                                                                                 // OPENCV
                c.fx = d(); c.fy = d(); c.cx = d(); c.cy = d();
                c.k1 = d(); c.k2 = d(); c.p1 = d(); c.p2 = d();
                break;
            default: throw std::runtime_error("Unsupported COLMAP camera model: " + std::to_string(c.model));
        }
        cams[id] = c;
    }
    return cams;
}

struct ColmapImage {
    uint32_t cam = 0;
    double q[4] = {1, 0, 0, 0}, t[3] = {0, 0, 0};
    std::string name;
};

std::vector<ColmapImage> read_images_bin(const std::string &path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open " + path);
    const uint64_t n = rd<uint64_t>(f);
    std::vector<ColmapImage> out;
    for (uint64_t i = 0; i < n; ++i) {
        ColmapImage im;
        (void)rd<uint32_t>(f);  // image id
        for (auto &v : im.q) v = rd<double>(f);
        for (auto &v : im.t) v = rd<double>(f);
        im.cam = rd<uint32_t>(f);
        char ch;
        while (f.get(ch) && ch != '\0') im.name += ch;
        const uint64_t np = rd<uint64_t>(f);
        f.seekg((std::streamoff)(np * 24), std::ios::cur);
        out.push_back(std::move(im));
    }
    return out;
}

// world-to-camera (q = w x y z, t) -> camera-to-world with the OpenGL flip
// of columns 1 and 2 (load_colmap.cpp:101-122)
void w2c_to_c2w(const double q[4], const double t[3], float out[16]) {
    double w = q[0], x = q[1], y = q[2], z = q[3];
    const double n = std::sqrt(w * w + x * x + y * y + z * z);
    w /= n;
    x /= n;
    y /= n;
    z /= n;
    const float R[9] = {(float)(1 - 2 * (y * y + z * z)), (float)(2 * (x * y - w * z)), (float)(2 * (x * z + w * y)),
                        (float)(2 * (x * y + w * z)), (float)(1 - 2 * (x * x + z * z)), (float)(2 * (y * z - w * x)),
                        (float)(2 * (x * z - w * y)), (float)(2 * (y * z + w * x)), (float)(1 - 2 * (x * x + y * y))};
    const float Ri[9] = {R[0], R[3], R[6], R[1], R[4], R[7], R[2], R[5], R[8]};
    float Ti[3];
    for (int r = 0; r < 3; ++r)
        Ti[r] = -(Ri[3 * r] * (float)t[0] + Ri[3 * r + 1] * (float)t[1] + Ri[3 * r + 2] * (float)t[2]);
    for (int r = 0; r < 3; ++r) {
        out[4 * r + 0] = Ri[3 * r];
        out[4 * r + 1] = -Ri[3 * r + 1];
        out[4 * r + 2] = -Ri[3 * r + 2];
        out[4 * r + 3] = Ti[r];
    }
    out[12] = out[13] = out[14] = 0.0f;
    out[15] = 1.0f;
}

InputData load_colmap(const std::string &root, const std::string &imageSource) {
    const fs::path r(root);
    const std::string sparse = fs::exists(r / "cameras.bin") ? root : (r / "sparse" / "0").string();
    const std::string imgdir = !imageSource.empty() ? imageSource : fs::exists(r / "images") ? (r / "images").string() : root;
    const auto cams = read_cameras_bin(sparse + "/cameras.bin");
    auto images = read_images_bin(sparse + "/images.bin");
    std::sort(images.begin(), images.end(), [](const ColmapImage &a, const ColmapImage &b) { return a.name < b.name; });
    InputData data;
    for (const auto &im : images) {
        auto it = cams.find(im.cam);
        if (it == cams.end()) continue;
        const ColmapCam &c = it->second;
        Camera cam;
        cam.width = c.width;
        cam.height = c.height;
        cam.fx = c.fx;
        cam.fy = c.fy;
        cam.cx = c.cx;
        cam.cy = c.cy;
        cam.k1 = c.k1;
        cam.k2 = c.k2;
        cam.p1 = c.p1;
        cam.p2 = c.p2;
        cam.filePath = imgdir + "/" + im.name;
        w2c_to_c2w(im.q, im.t, cam.camToWorld);
        data.cameras.push_back(std::move(cam));
    }
    if (fs::exists(sparse + "/points3D.bin"))
        data.points = readColmapPoints(sparse + "/points3D.bin");
    else if (fs::exists(sparse + "/points3D.ply"))
        data.points = readPly(sparse + "/points3D.ply");
    autoScaleAndCenter(data);
    return data;
}

// --------------------------------------------------------------- Polycam --

Camera polycam_frame(const Json &j) {
    Camera cam;
    cam.width = (int)j.value("width", 0.0);
    cam.height = (int)j.value("height", 0.0);
    cam.fx = (float)j.value("fx", 0.0);
    cam.fy = (float)j.value("fy", 0.0);
    cam.cx = (float)j.value("cx", cam.width / 2.0);
    cam.cy = (float)j.value("cy", cam.height / 2.0);
    return cam;
}

InputData load_polycam(const std::string &root) {
    const fs::path r(root), kf = r / "keyframes" / "corrected_cameras", imgs = r / "keyframes" / "corrected_images";
    InputData data;
    if (fs::exists(kf)) {
        std::vector<fs::path> files;
        for (auto &e : fs::directory_iterator(kf))
            if (e.path().extension() == ".json") files.push_back(e.path());
        std::sort(files.begin(), files.end());
        for (const auto &p : files) {
            const Json j = read_json(p);
            Camera cam = polycam_frame(j);
            float R[9];
            for (int a = 0; a < 3; ++a)
                for (int b = 0; b < 3; ++b) R[3 * a + b] = (float)j.value("R_" + std::to_string(a) + std::to_string(b), 0.0);
            const float T[3] = {(float)j.value("t_20", 0.0), (float)j.value("t_21", 0.0), (float)j.value("t_22", 0.0)};
            // rows 1 and 2 negated (load_polycam.cpp:47-51)
            for (int c = 0; c < 3; ++c) {
                cam.camToWorld[c] = R[c];
                cam.camToWorld[4 + c] = -R[3 + c];
                cam.camToWorld[8 + c] = -R[6 + c];
            }
            cam.camToWorld[3] = T[0];
            cam.camToWorld[7] = -T[1];
            cam.camToWorld[11] = -T[2];
            cam.camToWorld[15] = 1.0f;
            cam.filePath = resolve_image((imgs / p.stem()).string());
            data.cameras.push_back(std::move(cam));
        }
    } else {
        const Json j = read_json(r / "cameras.json");
        const Json &frames = j.has("frames") ? j.at("frames") : j;
        for (const Json &fr : frames.arr) {
            Camera cam = polycam_frame(fr);
            if (fr.has("transform_matrix")) read_matrix4(fr.at("transform_matrix"), cam.camToWorld);
            cam.filePath = fr.value("file_path", std::string());
            if (!cam.filePath.empty() && cam.filePath[0] != '/') cam.filePath = (r / cam.filePath).string();
            data.cameras.push_back(std::move(cam));
        }
    }
    for (const char *p : {"keyframes/point_cloud.ply", "point_cloud.ply", "sparse.ply"})
        if (fs::exists(r / p)) {
            data.points = readPly((r / p).string());
            break;
        }
    autoScaleAndCenter(data);
    return data;
}

// ------------------------------------------------------------------ PLY --

int ply_type_size(const std::string &t) {
    if (t == "char" || t == "uchar" || t == "int8" || t == "uint8") return 1;
    if (t == "short" || t == "ushort" || t == "int16" || t == "uint16") return 2;
    if (t == "int" || t == "uint" || t == "float" || t == "int32" || t == "uint32" || t == "float32") return 4;
    if (t == "double" || t == "float64") return 8;
    throw std::runtime_error("PLY: unknown property type " + t);
}

double ply_read(const uint8_t *p, const std::string &t) {
    if (t == "char" || t == "int8") return (double)*(const int8_t *)p;
    if (t == "uchar" || t == "uint8") return (double)*p;
    int16_t s;
    uint16_t us;
    int32_t i;
    uint32_t u;
    float f;
    double d;
    if (t == "short" || t == "int16") return std::memcpy(&s, p, 2), (double)s;
    if (t == "ushort" || t == "uint16") return std::memcpy(&us, p, 2), (double)us;
    if (t == "int" || t == "int32") return std::memcpy(&i, p, 4), (double)i;
    if (t == "uint" || t == "uint32") return std::memcpy(&u, p, 4), (double)u;
    if (t == "float" || t == "float32") return std::memcpy(&f, p, 4), (double)f;
    return std::memcpy(&d, p, 8), d;
}

}  // namespace

// Point cloud PLY (binary little-endian or ASCII): x y z and, when present,
// red green blue (uchar, or float in [0,1]) of the vertex element
// (load_ply.cpp:35-160).  Missing colours are mid-grey.
Points readPly(const std::string &path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("Cannot open PLY file: " + path);
    std::string line;
    std::getline(f, line);
    if (line.rfind("ply", 0) != 0) throw std::runtime_error("Not a PLY file: " + path);
    bool binary = false, ascii = false, in_vertex = false;
    int64_t n = 0;
    struct Prop {
        std::string name, type;
        int offset;
    };
    std::vector<Prop> props;
    int stride = 0;
    while (std::getline(f, line)) {
        if (!line.empty() && line.back() == '\r') line.pop_back();
        if (line == "end_header") break;
        std::istringstream is(line);
        std::string tok;
        is >> tok;
        if (tok == "format") {
            std::string fmt;
            is >> fmt;
            binary = fmt == "binary_little_endian";
            ascii = fmt == "ascii";
        } else if (tok == "element") {
            std::string name;
            is >> name;
            in_vertex = name == "vertex";
            if (in_vertex) is >> n;
        } else if (tok == "property" && in_vertex) {
            std::string type, name;
            is >> type >> name;
            if (type == "list") throw std::runtime_error("PLY: list properties in the vertex element");
            props.push_back({name, type, stride});
            stride += ply_type_size(type);
        }
    }
    if (!binary && !ascii) throw std::runtime_error("PLY: unsupported format in " + path);
    auto find = [&](std::initializer_list<const char *> names) -> int {
        for (const char *nm : names)
            for (size_t i = 0; i < props.size(); ++i)
                if (props[i].name == nm) return (int)i;
        return -1;
    };
    const int ix = find({"x"}), iy = find({"y"}), iz = find({"z"});
    const int ir = find({"red", "r"}), ig = find({"green", "g"}), ib = find({"blue", "b"});
    if (ix < 0 || iy < 0 || iz < 0) throw std::runtime_error("PLY: vertex has no x/y/z");
    Points pts;
    pts.count = n;
    pts.xyz.resize((size_t)n * 3);
    pts.rgb.assign((size_t)n * 3, 128);
    std::vector<uint8_t> row((size_t)stride);
    std::vector<double> vals(props.size());
    for (int64_t i = 0; i < n; ++i) {
        if (binary) {
            f.read((char *)row.data(), stride);
            if (!f) throw std::runtime_error("PLY: truncated vertex data in " + path);
            for (size_t k = 0; k < props.size(); ++k) vals[k] = ply_read(row.data() + props[k].offset, props[k].type);
        } else {
            for (auto &v : vals)
                if (!(f >> v)) throw std::runtime_error("PLY: truncated ASCII vertex data in " + path);
        }
        pts.xyz[3 * i] = (float)vals[ix];
        pts.xyz[3 * i + 1] = (float)vals[iy];
        pts.xyz[3 * i + 2] = (float)vals[iz];
        const int ic[3] = {ir, ig, ib};
        for (int c = 0; c < 3; ++c)
            if (ic[c] >= 0) {
                const bool fl = props[ic[c]].type.rfind("float", 0) == 0 || props[ic[c]].type == "double";
                const double v = fl ? vals[ic[c]] * 255.0 : vals[ic[c]];
                pts.rgb[3 * i + c] = (uint8_t)std::min(255.0, std::max(0.0, v));
            }
    }
    return pts;
}

Points readColmapPoints(const std::string &path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("Cannot open points3D.bin: " + path);
    const uint64_t n = rd<uint64_t>(f);
    Points pts;
    pts.count = (int64_t)n;
    pts.xyz.resize(n * 3);
    pts.rgb.resize(n * 3);
    for (uint64_t i = 0; i < n; ++i) {
        (void)rd<uint64_t>(f);
        for (int k = 0; k < 3; ++k) pts.xyz[3 * i + k] = (float)rd<double>(f);
        for (int k = 0; k < 3; ++k) pts.rgb[3 * i + k] = rd<uint8_t>(f);
        (void)rd<double>(f);
        const uint64_t track = rd<uint64_t>(f);
        f.seekg((std::streamoff)(track * 8), std::ios::cur);
    }
    return pts;
}

InputData inputDataFromX(const std::string &path, const std::string &colmapImagePath) {
    const fs::path root(path);
    InputData data;
    if (fs::exists(root / "transforms.json"))
        data = load_nerfstudio(path);
    else if (fs::exists(root / "cameras.bin") || fs::exists(root / "sparse" / "0" / "cameras.bin"))
        data = load_colmap(path, colmapImagePath);
    else if (fs::exists(root / "keyframes" / "corrected_cameras") || fs::exists(root / "cameras.json"))
        data = load_polycam(path);
    else
        throw std::runtime_error("Unrecognized dataset format in: " + path +
                                 "\nSupported: COLMAP (cameras.bin), Nerfstudio (transforms.json), Polycam (keyframes/)");
    if (data.cameras.empty()) throw std::runtime_error("dataset has no cameras: " + path);
    if (data.points.count == 0) {
        std::cerr << "msplat: no SfM point cloud found, seeding camera-aware random init\n";
        initializeRandomPointsCameraAware(data, 100000, 0.35f);
    }
    return data;
}
