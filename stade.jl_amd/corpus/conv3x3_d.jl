function conv3x3_d(loss, lossd, xp, xpd, w, wd, out, outd, i_nb, i_c, i_k, i_h, i_w)
    i_wp = i_w + 2
    i_hp = i_h + 2
    for idx = 1:i_nb * i_k * i_h * i_w
        __icse_0 = idx - 1
        i_x = mod(__icse_0, i_w) + 1
        i_y = mod(div(__icse_0, i_w), i_h) + 1
        i_co = mod(div(__icse_0, i_w * i_h), i_k) + 1
        i_n = div(__icse_0, i_w * i_h * i_k) + 1
        sd = 0.0
        s = 0.0
        for i_t = 1:i_c * 9
            __icse_1 = i_t - 1
            i_ci = div(__icse_1, 9) + 1
            i_ky = mod(div(__icse_1, 3), 3) + 1
            i_kx = mod(__icse_1, 3) + 1
            __icse_2 = ((i_co - 1) * i_c + (i_ci - 1)) * 9 + (i_ky - 1) * 3 + i_kx
            __icse_3 = (((i_n - 1) * i_c + (i_ci - 1)) * i_hp + (i_y + i_ky - 2)) * i_wp + i_x + i_kx - 1
            __cse_4 = xp[__icse_3]
            __cse_5 = w[__icse_2]
            sd = sd + (__cse_4 * wd[__icse_2] + __cse_5 * xpd[__icse_3])
            s = s + __cse_5 * __cse_4
        end
        outd[idx] = sd
        out[idx] = s
    end
    for i_q = 1:i_nb * i_k * i_h * i_w
        __cse_6 = out[i_q]
        lossd[1] = lossd[1] + 0.5 * ((2__cse_6) * outd[i_q])
        loss[1] = loss[1] + 0.5 * __cse_6 ^ 2
    end
    return nothing
end

function conv3x3(loss, xp, w, out, i_nb, i_c, i_k, i_h, i_w)
    i_wp = i_w + 2
    i_hp = i_h + 2
    # one iteration per output pixel (x, y, output channel, sample); the tap sum is carried (rule 1)
    for idx = 1:i_nb * i_k * i_h * i_w
        i_x = mod(idx - 1, i_w) + 1
        i_y = mod(div(idx - 1, i_w), i_h) + 1
        i_co = mod(div(idx - 1, i_w * i_h), i_k) + 1
        i_n = div(idx - 1, i_w * i_h * i_k) + 1
        s = 0.0
        for i_t = 1:i_c * 9
            i_ci = div(i_t - 1, 9) + 1
            i_ky = mod(div(i_t - 1, 3), 3) + 1
            i_kx = mod(i_t - 1, 3) + 1
            s = s + w[((i_co - 1) * i_c + (i_ci - 1)) * 9 + (i_ky - 1) * 3 + i_kx] * xp[(((i_n - 1) * i_c + (i_ci - 1)) * i_hp + (i_y + i_ky - 2)) * i_wp + i_x + i_kx - 1]
        end
        out[idx] = s
    end
    # half the squared norm of the output
    for i_q = 1:i_nb * i_k * i_h * i_w
        loss[1] = loss[1] + 0.5 * out[i_q] ^ 2
    end
    return nothing
end
